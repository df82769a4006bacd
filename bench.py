"""Benchmark of the MI355X DSA path (one GPU).

A step is one sparse-MLA forward over the prefill workload
C4 (B=1, Sq=Skv=16384, H=128, d_qk=576, d_v=512, topk=2048, bf16, causal
indices with -1 padding), timed with HIP events on the launch stream.  The same
run also measures the lightning indexer + top-k (config C2: 4096 x 32768, 64
fp8 heads x 128, top-2048) and the paged sparse-MLA decode (config C3: B=64,
H=128, topk=2048 over a 64K-token paged cache), each with an L2/MALL flush
before every repetition, and times the CPU oracle on a bounded sample of the
step workload as the reported CPU baseline.

Prints one JSON line (see the keys below).  Synthetic inputs, seeded.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_BF16_TFLOPS = 2500.0
PEAK_FP8_TFLOPS = 5000.0
PEAK_HBM_GBS = 8000.0


def _log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


class _Flush:
    """Cold caches before a timed call: zero a 512 MiB buffer (the reference's L2 flush,
    tilelang/profiler/bench.py:46-52, sized past MI355X's 256 MB MALL), then read a second 512 MiB
    buffer.  The read evicts the zero-fill's dirty lines -- their write-back happens here, not
    inside the timed call -- and leaves L2 and MALL holding clean, unrelated lines.  `zero_only`
    skips the read (the reference's flush alone; C3 decode reports both)."""

    def __init__(self, torch, dev):
        self.fill = torch.empty(512 * 1024 * 1024 // 4, dtype=torch.float32, device=dev)
        self.drain = torch.ones(512 * 1024 * 1024 // 4, dtype=torch.float32, device=dev)
        self.zero_only = False

    def zero_(self):
        self.fill.zero_()
        if not self.zero_only:
            self.drain.max()


def _flush_buffer(torch, dev):
    return _Flush(torch, dev)


def _timed(torch, fn, reps, flush=None):
    """Per-rep device time (ms) from HIP events on the current stream; optional cache flush before each rep."""
    times = []
    for _ in range(reps):
        if flush is not None:
            flush.zero_()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        fn()
        e1.record()
        e1.synchronize()
        times.append(e0.elapsed_time(e1))
    return times


def _timed_graph(torch, fn, n):
    """Device time (ms) per call: n calls captured in one HIP graph, the replay timed with HIP
    events -- what the device spends per call, without the host's per-call submission cost."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(n):
            fn()
    graph.replay()
    torch.cuda.synchronize()
    times = []
    for _ in range(5):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        graph.replay()
        e1.record()
        e1.synchronize()
        times.append(e0.elapsed_time(e1) / n)
    del graph
    return _median(times)


def _median(x):
    s = sorted(x)
    return s[len(s) // 2]


def gen_prefill(torch, dev, S=16384, H=128, topk=2048, seed=20261204):
    """C4: q, kv ~ N(0,1)*0.5 bf16; row i draws min(topk, i+1) distinct indices from [0, i], -1 padded."""
    g = torch.Generator(device=dev).manual_seed(seed)
    q = (torch.randn(1, S, H, 576, generator=g, device=dev) * 0.5).to(torch.bfloat16)
    kv = (torch.randn(1, S, 1, 576, generator=g, device=dev) * 0.5).to(torch.bfloat16)
    idx = torch.empty(1, S, 1, topk, dtype=torch.int32, device=dev)
    cols = torch.arange(S, device=dev).view(1, -1)
    for r0 in range(0, S, 2048):
        r1 = min(S, r0 + 2048)
        u = torch.rand(r1 - r0, S, generator=g, device=dev)
        u = torch.where(cols <= torch.arange(r0, r1, device=dev).view(-1, 1), u, torch.full_like(u, -1.0))
        v, i = torch.topk(u, topk, dim=1)
        idx[0, r0:r1, 0] = torch.where(v >= 0, i, torch.full_like(i, -1)).to(torch.int32)
        del u, v, i
    return q, kv, idx


def gen_decode(torch, dev, B=64, ctx=65536, H=128, topk=2048, bs=64, seed=20261203):
    """C3: paged pool of B*ctx/bs blocks, seeded random block table, topk distinct indices per sequence."""
    g = torch.Generator(device=dev).manual_seed(seed)
    nblk = ctx // bs
    q = (torch.randn(B, 1, H, 576, generator=g, device=dev) * 0.5).to(torch.bfloat16)
    pool = (torch.randn(B * nblk, bs, 1, 576, generator=g, device=dev) * 0.5).to(torch.bfloat16)
    table = torch.randperm(B * nblk, generator=g, device=dev).view(B, nblk).to(torch.int32)
    u = torch.rand(B, ctx, generator=g, device=dev)
    idx = torch.topk(u, topk, dim=1).indices.to(torch.int32).view(B, 1, 1, topk)
    lens = torch.full((B,), ctx, dtype=torch.int32, device=dev)
    return q, pool, table, idx, lens


def gen_indexer(torch, dev, S1=4096, S2=32768, H=64, D=128, seed=20261202):
    """C2: q = fp8(N(0,1)); k fp8 per-token with scale absmax/448; w ~ N(0,1)/8."""
    g = torch.Generator(device=dev).manual_seed(seed)
    q = torch.randn(1, S1, H, D, generator=g, device=dev).to(torch.float8_e4m3fn)
    kf = torch.randn(1, S2, D, generator=g, device=dev)
    amax = kf.abs().amax(dim=-1)
    ks = (amax / 448.0).to(torch.float32)
    k = (kf / ks.unsqueeze(-1)).clamp(-448, 448).to(torch.float8_e4m3fn).unsqueeze(2).contiguous()
    w = torch.randn(1, S1, H, generator=g, device=dev) / 8
    return q, k, w, ks


def cpu_baseline_prefill(torch, q, kv, idx, budget_s=12.0):
    """The oracle (fp32) on the last query rows of the C4 workload, until ~budget_s of CPU time."""
    from oracle import dsa_oracle as ref

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    S = q.shape[1]
    H = q.shape[2]
    rows = 0
    t0 = time.perf_counter()
    step = 4
    while time.perf_counter() - t0 < budget_s and rows + step <= S:
        r1 = S - rows
        r0 = r1 - step
        qs = q[:, r0:r1].cpu()
        ids = idx[:, r0:r1].cpu()
        kvs = kv[:, :r1].cpu()
        ref.sparse_mla_fwd(qs, kvs, ids, 576 ** -0.5, actual_seq_lengths_query=[step],
                           actual_seq_lengths_kv=[r1], compute_dtype=torch.float32)
        rows += step
    el = time.perf_counter() - t0
    flops = 2.0 * H * idx.shape[-1] * (576 + 512) * rows
    return {"value": flops / el / 1e12, "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": f"oracle sparse_mla_fwd (torch fp32 gather/softmax) on the last {rows} of {S} query rows "
                      f"of the step workload, {el:.1f} s"}


def _cpu_model():
    """The host CPU as /proc/cpuinfo names it: model name, family / model / stepping (which tell the
    generation where a VM reports only "AMD EPYC"), clock, logical CPUs and AVX-512 support."""
    info = {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if not line.strip():
                    break  # first processor entry only
                key, _, val = line.partition(":")
                info[key.strip()] = val.strip()
    except OSError:
        pass
    import platform

    name = info.get("model name") or platform.processor() or "unknown"
    fields = [name]
    if "cpu family" in info:
        fields.append(f"family {info['cpu family']} model {info.get('model', '?')} stepping {info.get('stepping', '?')}")
    if "cpu MHz" in info:
        fields.append(f"{float(info['cpu MHz']):.0f} MHz")
    fields.append(f"{os.cpu_count()} logical CPUs")
    if "flags" in info:
        fields.append("avx512f" if "avx512f" in info["flags"].split() else "no avx512f")
    return ", ".join(fields)


def cpu_baselines_other(torch):
    """The oracle (fp32, all host threads) on the other configurations: C1 at full shape, C2 and C3 on
    bounded samples scaled linearly to the full shape (labelled "extrapolated")."""
    from oracle import dsa_oracle as ref

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    res = {}

    # C1: B=1, Sq=128, Skv=4096, H=16, topk=512, the parity case's own inputs (seed 20261201).
    g = torch.Generator().manual_seed(20261201)
    q = (torch.randn(1, 128, 16, 576, generator=g) * 0.5).to(torch.bfloat16)
    kv = (torch.randn(1, 4096, 1, 576, generator=g) * 0.5).to(torch.bfloat16)
    idx = ref.causal_sparse_indices(1, 128, 4096, 512, seed=20261201)
    ref.sparse_mla_fwd(q[:, :4], kv, idx[:, :4], 576 ** -0.5, compute_dtype=torch.float32)  # warm
    t0 = time.perf_counter()
    ref.sparse_mla_fwd(q, kv, idx, 576 ** -0.5, compute_dtype=torch.float32)
    el = time.perf_counter() - t0
    fl = 2.0 * 16 * 512 * 1088 * 128
    res["C1_sparse_mla"] = {"value": round(fl / el / 1e12, 4), "unit": "TFLOP/s", "ms": round(el * 1e3, 1),
                            "sample": "full shape (128 queries x 16 heads x topk 512 over 4096 keys)"}

    # C2: indexer logits + top-2048 over the last 256 of 4096 query rows (32768 keys, 64 fp8 heads x 128), x16.
    g = torch.Generator().manual_seed(20261202)
    S1, S2, Hi, D, K, rows = 4096, 32768, 64, 128, 2048, 256
    qi = torch.randn(1, rows, Hi, D, generator=g).to(torch.float8_e4m3fn)
    kf = torch.randn(1, S2, D, generator=g)
    ks = (kf.abs().amax(dim=-1) / 448.0).to(torch.float32)
    ki = (kf / ks.unsqueeze(-1)).clamp(-448, 448).to(torch.float8_e4m3fn)
    wi = torch.randn(1, rows, Hi, generator=g) / 8
    del kf
    t0 = time.perf_counter()
    # The last 256 rows of the causal chunk see keys s <= S2 - S1 + t: as rows of a 256-row chunk at the tail.
    lg = ref.indexer_logits(qi, ki, wi, ks, sparse_mode=3, row_chunk=16, compute_dtype=torch.float32)
    t1 = time.perf_counter()
    ref.topk_stable(lg.view(rows, S2), K)
    t2 = time.perf_counter()
    scale = S1 / rows
    res["C2_indexer_topk"] = {"us": round((t2 - t0) * scale * 1e6, 0), "indexer_us": round((t1 - t0) * scale * 1e6, 0),
                              "topk_us": round((t2 - t1) * scale * 1e6, 0), "unit": "us per call",
                              "sample": f"last {rows} of {S1} query rows, x{scale:.0f} (extrapolated)"}
    del qi, ki, wi, lg

    # C3: paged decode, 8 of the 64 sequences (their 1024 blocks each, remapped), x8.
    g = torch.Generator().manual_seed(20261203)
    nseq, B, H, bs, nblk, topk = 8, 64, 128, 64, 1024, 2048
    qd = (torch.randn(nseq, 1, H, 576, generator=g) * 0.5).to(torch.bfloat16)
    pool = (torch.randn(nseq * nblk, bs, 1, 576, generator=g) * 0.5).to(torch.bfloat16)
    table = torch.randperm(nseq * nblk, generator=g).view(nseq, nblk).to(torch.int32)
    idd = torch.stack([torch.randperm(nblk * bs, generator=g)[:topk] for _ in range(nseq)]).to(torch.int32)
    idd = idd.view(nseq, 1, 1, topk)
    t0 = time.perf_counter()
    ref.sparse_mla_fwd(qd, pool, idd, 576 ** -0.5, block_table=table, compute_dtype=torch.float32)
    el = (time.perf_counter() - t0) * (B / nseq)
    res["C3_decode"] = {"us": round(el * 1e6, 0), "unit": "us per call",
                        "sample": f"{nseq} of {B} sequences (128 heads x topk 2048, 64-token blocks), x{B // nseq} "
                                  "(extrapolated)"}
    res["cores"] = threads
    res["kind"] = "port"
    return res


def run_step(torch, pkg, dev, args, S, H, topk, sm_scale, flush):
    """C4 sparse MLA prefill: the timed step, each behind the cache flush the other parts use
    (tilelang/profiler/bench.py:46-52 zero-fills a buffer before each rep).  Returns (result dict,
    inputs for the CPU baseline)."""
    _log("generating C4 prefill inputs")
    q, kv, idx = gen_prefill(torch, dev, S=S, H=H, topk=topk)
    fn = lambda: pkg.sparse_mla_fwd(q, kv, idx, sm_scale)  # noqa: E731
    # Warmup behind the same flush: the flush buffers' first use would otherwise land in the timed steps.
    _timed(torch, fn, args.warmup, flush)
    torch.cuda.synchronize()
    _log(f"C4 warmup done; timing {args.steps} steps")
    t0 = time.perf_counter()
    step_ms = _timed(torch, fn, args.steps, flush)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = sum(step_ms) / len(step_ms)
    flops = 2.0 * H * topk * (576 + 512) * S
    tflops = flops / (ms * 1e-3) / 1e12
    _log(f"C4 sparse MLA prefill: {ms:.3f} ms/step, {tflops:.1f} TFLOP/s")
    result = {
        "metric": "sparse-MLA TFLOPS (% MFMA peak) + indexer/top-k µs @H=128, topk=2048",
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1)*0.5 bf16 q/kv, causal uniform indices)",
        "timing": "HIP events around each step, a 512 MB zero-fill + 512 MB read flush before each",
        "config": {"workload": "C4 sparse MLA prefill", "batch": 1, "seq_len_q": S, "seq_len_kv": S, "heads": H,
                   "d_qk": 576, "d_v": 512, "topk": topk, "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tflops / PEAK_BF16_TFLOPS, 4),
                     # HBM bytes per launch from the committed FETCH_SIZE/WRITE_SIZE summary; at H=128 the
                     # kernel runs one 256-thread workgroup per query token.
                     "traffic": profiled_traffic(STEP_KERNEL, S * 256),
                     "traffic_source": "profiles/traffic_c4_prefill_step.txt",
                     "kernel": STEP_KERNEL, "flops_per_launch": flops},
        "wall_s_timed_region": round(wall, 4),
        "step_ms_p10_p90": [round(sorted(step_ms)[len(step_ms) // 10], 4),
                            round(sorted(step_ms)[(len(step_ms) * 9) // 10], 4)],
    }
    return result, (q, kv, idx)


C5_SEED = 20261205


def gen_c5_prefill(torch, dev, g, ctx=131072, chunk=4096, H=128, Hi=64, D=128):
    """C5 prefill chunk (the last `chunk` of `ctx` positions): fp8 indexer q [1, chunk, Hi, D], keys
    [1, ctx, D] fp8 with per-token scale absmax/448, weights N(0,1)/8; MLA q [1, chunk, H, 576] and
    kv [1, ctx, 1, 576] bf16 ~ N(0,1)*0.5.  Draws from generator `g` in that order."""
    qi = torch.randn(1, chunk, Hi, D, generator=g, device=dev).to(torch.float8_e4m3fn)
    kf = torch.randn(1, ctx, D, generator=g, device=dev)
    ks = (kf.abs().amax(dim=-1) / 448.0).to(torch.float32)
    ki = (kf / ks.unsqueeze(-1)).clamp(-448, 448).to(torch.float8_e4m3fn).contiguous()
    del kf
    wi = torch.randn(1, chunk, Hi, generator=g, device=dev) / 8
    q = (torch.randn(1, chunk, H, 576, generator=g, device=dev) * 0.5).to(torch.bfloat16)
    kv = (torch.randn(1, ctx, 1, 576, generator=g, device=dev) * 0.5).to(torch.bfloat16)
    return qi, ki, ks, wi, q, kv


def gen_c5_decode(torch, dev, g, ctx=131072, dec_b=32, H=128, Hi=64, D=128, bs=64):
    """C5 decode step: `dec_b` sequences x 1 query over `ctx` keys each, paged in `bs`-token blocks
    behind one seeded random block table shared by the fp8 index keys and the bf16 latent KV pool.
    Draws from generator `g` (after gen_c5_prefill in the benchmark)."""
    nblk = ctx // bs
    qd = torch.randn(dec_b, 1, Hi, D, generator=g, device=dev).to(torch.float8_e4m3fn)
    kdf = torch.randn(dec_b * nblk, bs, D, generator=g, device=dev)
    kds = (kdf.abs().amax(dim=-1) / 448.0).to(torch.float32)
    kd = (kdf / kds.unsqueeze(-1)).clamp(-448, 448).to(torch.float8_e4m3fn).contiguous()
    del kdf
    wd = torch.randn(dec_b, 1, Hi, generator=g, device=dev) / 8
    table = torch.randperm(dec_b * nblk, generator=g, device=dev).view(dec_b, nblk).to(torch.int32)
    lens_q = torch.ones(dec_b, dtype=torch.int32, device=dev)
    lens_k = torch.full((dec_b,), ctx, dtype=torch.int32, device=dev)
    qm = (torch.randn(dec_b, 1, H, 576, generator=g, device=dev) * 0.5).to(torch.bfloat16)
    pool = (torch.randn(dec_b * nblk, bs, 1, 576, generator=g, device=dev) * 0.5).to(torch.bfloat16)
    return qd, kd, kds, wd, table, lens_q, lens_k, qm, pool


def run_c5(torch, pkg, dev, args, flush, ctx=131072, chunk=4096, H=128, topk=2048, dec_b=32):
    """C5: one sequence of 128K keys; a prefill chunk of 4096 queries at its tail runs indexer -> top-k ->
    sparse MLA on the indexer's own selection; then a decode step of 32 sequences (one query each, 128K keys
    each, paged 64-token blocks) through the same three kernels."""
    from tilelang_ascend_amd import _lib as L

    lib = pkg.load_library()
    stream = L.stream_handle(dev)
    _log("C5 inputs")
    g = torch.Generator(device=dev).manual_seed(C5_SEED)
    Hi, D = 64, 128
    qi, ki, ks, wi, q, kv = gen_c5_prefill(torch, dev, g, ctx=ctx, chunk=chunk, H=H, Hi=Hi, D=D)
    logits = torch.empty(chunk, ctx, dtype=torch.float32, device=dev)
    idx = torch.empty(1, chunk, 1, topk, dtype=torch.int32, device=dev)
    out = torch.empty(1, chunk, H, 512, dtype=torch.bfloat16, device=dev)
    lse = torch.empty(1, chunk, H, dtype=torch.float32, device=dev)
    ws_b = lib.dsa_sparse_mla_workspace_size(1, chunk, H, topk)
    ws = torch.empty(max(ws_b, 1), dtype=torch.uint8, device=dev)
    sm = 576 ** -0.5

    def run_idx():
        L.check(lib.dsa_indexer_logits(L.KIND_FP8_E4M3, qi.data_ptr(), ki.data_ptr(), ks.data_ptr(), wi.data_ptr(), 1,
                                       chunk, ctx, Hi, D, None, None, None, 0, 0, 3, logits.data_ptr(), ctx, stream),
                "c5 indexer")

    tws_b = lib.dsa_topk_select_workspace_size(chunk, ctx, topk)
    tws = torch.empty(max(tws_b, 1), dtype=torch.uint8, device=dev)

    def run_topk():
        L.check(lib.dsa_topk_select_ws(logits.data_ptr(), ctx, chunk, ctx, topk, None, 1, idx.data_ptr(), None,
                                       tws.data_ptr(), tws_b, stream), "c5 topk")

    def run_mla():
        L.check(lib.dsa_sparse_mla_fwd(L.KIND_BF16, q.data_ptr(), kv.data_ptr(), idx.data_ptr(), None, None, None, 1,
                                       chunk, H, 576, 512, ctx, 0, 0, topk, sm, 1, out.data_ptr(), lse.data_ptr(),
                                       ws.data_ptr(), ws_b, stream), "c5 mla")

    fidx = torch.empty(1, chunk, 1, topk, dtype=torch.int32, device=dev)
    fws_b = lib.dsa_lightning_indexer_fused_workspace_size(1, chunk, ctx, topk)
    fws = torch.empty(fws_b, dtype=torch.uint8, device=dev)
    fcnt = torch.zeros(1, dtype=torch.int32, device=dev)

    def run_fused():
        L.check(lib.dsa_lightning_indexer_fused(L.KIND_FP8_E4M3, qi.data_ptr(), ki.data_ptr(), ks.data_ptr(),
                                                wi.data_ptr(), 1, chunk, ctx, Hi, D, None, None, None, 0, 0, 3, topk,
                                                fidx.data_ptr(), None, fws.data_ptr(), fws_b, stream), "c5 fused")

    for f in (run_idx, run_topk, run_mla, run_fused):
        f()
    L.check(lib.dsa_lightning_indexer_fused_fallback_rows(fws.data_ptr(), 1, chunk, ctx, topk, fcnt.data_ptr(),
                                                          stream), "c5 fallback rows")
    torch.cuda.synchronize()
    fused_same = bool(torch.equal(fidx, idx))
    fused_fallback = int(fcnt.item())
    reps = max(3, args.reps // 2)
    t_idx = _median(_timed(torch, run_idx, reps, flush))
    t_topk = _median(_timed(torch, run_topk, reps, flush))
    t_mla = _median(_timed(torch, run_mla, reps, flush))
    t_fused = _median(_timed(torch, run_fused, reps, flush))
    del fws
    pairs = sum(min(ctx, ctx - chunk + t + 1) for t in range(chunk))
    idx_flops = 2.0 * Hi * D * chunk * ctx
    mla_flops = 2.0 * H * topk * (576 + 512) * chunk
    topk_bytes = chunk * ctx * 4 + chunk * topk * 4
    roof_us = (idx_flops / (PEAK_FP8_TFLOPS * 1e12) + topk_bytes / (PEAK_HBM_GBS * 1e9)) * 1e6
    floor_us = idx_flops / (PEAK_FP8_TFLOPS * 1e12) * 1e6
    del qi, ki, wi, logits, q, kv, out, lse, ws, tws

    # Decode step: 32 sequences x 1 query, 128K keys each, paged KV (64-token blocks).
    _log("C5 decode inputs")
    bs = 64
    nblk = ctx // bs
    qd, kd, kds, wd, table, lens_q, lens_k, qm, pool = gen_c5_decode(torch, dev, g, ctx=ctx, dec_b=dec_b, H=H, Hi=Hi,
                                                                     D=D, bs=bs)
    dlog = torch.empty(dec_b, 1, ctx, dtype=torch.float32, device=dev)
    didx = torch.empty(dec_b, 1, 1, topk, dtype=torch.int32, device=dev)
    dout = torch.empty(dec_b, 1, H, 512, dtype=torch.bfloat16, device=dev)
    dlse = torch.empty(dec_b, 1, H, dtype=torch.float32, device=dev)
    dws_b = lib.dsa_sparse_mla_workspace_size(dec_b, 1, H, topk)
    dws = torch.empty(max(dws_b, 1), dtype=torch.uint8, device=dev)

    dtws_b = lib.dsa_topk_select_workspace_size(dec_b, ctx, topk)
    dtws = torch.empty(max(dtws_b, 1), dtype=torch.uint8, device=dev)

    def run_decode():
        L.check(lib.dsa_indexer_logits(L.KIND_FP8_E4M3, qd.data_ptr(), kd.data_ptr(), kds.data_ptr(), wd.data_ptr(),
                                       dec_b, 1, ctx, Hi, D, lens_q.data_ptr(), lens_k.data_ptr(), table.data_ptr(),
                                       bs, nblk, 3, dlog.data_ptr(), ctx, stream), "c5 decode indexer")
        L.check(lib.dsa_topk_select_ws(dlog.data_ptr(), ctx, dec_b, ctx, topk, None, 1, didx.data_ptr(), None,
                                       dtws.data_ptr(), dtws_b, stream), "c5 decode topk")
        L.check(lib.dsa_sparse_mla_fwd(L.KIND_BF16, qm.data_ptr(), pool.data_ptr(), didx.data_ptr(), table.data_ptr(),
                                       lens_q.data_ptr(), lens_k.data_ptr(), dec_b, 1, H, 576, 512, ctx, bs, nblk,
                                       topk, sm, 1, dout.data_ptr(), dlse.data_ptr(), dws.data_ptr(), dws_b, stream),
                "c5 decode mla")

    run_decode()
    torch.cuda.synchronize()
    t_dec = _median(_timed(torch, run_decode, reps, flush))
    dec_bytes = dec_b * (ctx * (D + 4) + topk * 576 * 2 + H * 576 * 2 + H * 512 * 2) + dec_b * ctx * 4 * 2
    _log(f"C5: indexer {t_idx * 1e3:.1f} us, topk {t_topk * 1e3:.1f} us, fused {t_fused * 1e3:.1f} us "
         f"(same: {fused_same}, fallback rows {fused_fallback}), mla {t_mla * 1e3:.1f} us, "
         f"decode chain {t_dec * 1e3:.1f} us")
    del qd, kd, kds, wd, table, dlog, didx, qm, pool, dout, dlse, dws, dtws
    return {
        "workload": "C5: 4096-query chunk at the tail of a 128K context (fp8 indexer 64x128 -> top-2048 -> sparse "
                    "MLA H=128 on that selection), plus a decode step of 32 sequences x 128K keys",
        "indexer_us": round(t_idx * 1e3, 1),
        "topk_us": round(t_topk * 1e3, 1),
        "dense_indexer_topk_us": round((t_idx + t_topk) * 1e3, 1),
        "indexer_topk_us": round(t_fused * 1e3, 1),
        "indexer_topk_path": "fused (lightning_indexer streams the top-k for rows over 32768 keys)",
        "indexer_topk_roofline_us": round(roof_us, 1),
        "indexer_topk_frac_roofline": round(roof_us / (t_fused * 1e3), 4),
        "dense_frac_roofline": round(roof_us / ((t_idx + t_topk) * 1e3), 4),
        # The fused path never writes the logits, so its floor is the fp8 MFMA work alone.
        "fused_floor_us": round(floor_us, 1),
        "fused_frac_fp8_floor": round(floor_us / (t_fused * 1e3), 4),
        "indexer_tflops_dense": round(idx_flops / (t_idx * 1e-3) / 1e12, 1),
        "indexer_frac_fp8_peak": round(idx_flops / (t_idx * 1e-3) / 1e12 / PEAK_FP8_TFLOPS, 4),
        "indexer_causal_pair_frac": round(pairs / (chunk * ctx), 4),
        "fused_equals_dense": fused_same,
        "fused_fallback_rows": fused_fallback,
        "mla_us": round(t_mla * 1e3, 1),
        "mla_tflops": round(mla_flops / (t_mla * 1e-3) / 1e12, 1),
        "decode_chain_us": round(t_dec * 1e3, 1),
        "decode_chain_bytes": dec_bytes,
    }


PROFILES = ROOT / "profiles"
STEP_KERNEL = "dsa::sparse_mla_kernel<4, false, 576, false>"
COPY_KERNEL = "__amd_rocclr_copyBuffer"


# Published device times of the reference's V4 sparse_flash_mla (TileLang on Ascend, msprof task
# duration; examples/deepseek_v4/sparse_flash_mla/bench_mark.md), for the same shapes.
V4_REFERENCE_US = {"swa_prefill": 1490.930, "hca_prefill": 3141.853, "csa_prefill": 6022.700,
                   "swa_decode": 13.824, "hca_decode": 18.644, "csa_decode": 31.659}


def run_v4(torch, pkg, dev, args, flush, H=64, D=512, bs=128, K=512, win=127):
    """V4 sparse flash MLA at the reference benchmark's shapes (bench_mark.md: B=1, N1=64, D=512,
    TND, bf16, block 128, window 127, K=512, cmp_ratio 4 (swa/csa) / 128 (hca); prefill S=8192,
    decode one row against 8193 keys), through the C ABI on preallocated buffers.  Timed as the
    reference times it (repeated launches, no cache flush between them: msprof task duration with
    the first launch dropped): device time per call from a HIP graph of 20 calls (the host's
    per-call submission cost, larger than a decode step's device time, stays out, as it does
    from the reference's task durations), so the figures compare with V4_REFERENCE_US."""
    from tilelang_ascend_amd import _lib as L
    lib = pkg.load_library()
    g = torch.Generator(device=dev).manual_seed(20261205)
    res = {"workload": "V4 sparse_flash_mla, B=1, N1=64, D=512, bf16, 128-row blocks, window 127, K=512, "
                       "cmp_ratio 4 (swa, csa) / 128 (hca); prefill S=Skv=8192, decode 1 row x 8193 keys; "
                       "device time per call (HIP graph of 20 warm calls), as the reference's task durations"}
    for S, Skv, tag in ((8192, 8192, "prefill"), (1, 8193, "decode")):
        q = (torch.randn((S, H, D), device=dev, generator=g) * 0.5).to(torch.bfloat16)
        nb = (Skv + bs - 1) // bs
        ori = (torch.randn((nb, bs, 1, D), device=dev, generator=g) * 0.5).to(torch.bfloat16)
        obt = torch.randperm(nb, device=dev, generator=g).to(torch.int32).view(1, nb)
        sinks = torch.randn(H, device=dev, generator=g)
        qs = torch.zeros(1, dtype=torch.int32, device=dev)
        ql = torch.full((1,), S, dtype=torch.int32, device=dev)
        kl = torch.full((1,), Skv, dtype=torch.int32, device=dev)
        out = torch.empty((S, H, D), dtype=torch.bfloat16, device=dev)
        lse = torch.empty((S, H), dtype=torch.float32, device=dev)
        for mode, ratio in (("swa", 4), ("hca", 128), ("csa", 4)):
            ncmp = Skv // ratio
            cmp = cbt = idx = None
            if mode != "swa":
                cnb = max(1, (ncmp + bs - 1) // bs)
                cmp = (torch.randn((cnb, bs, 1, D), device=dev, generator=g) * 0.5).to(torch.bfloat16)
                cbt = torch.randperm(cnb, device=dev, generator=g).to(torch.int32).view(1, cnb)
            sg = torch.arange(S, device=dev) + (Skv - S)
            thr = (sg + 1) // ratio
            if mode == "csa":
                # Row s selects min(K, thr) distinct compressed rows below its threshold, -1 padded.
                u = torch.rand((S, max(ncmp, 1)), device=dev, generator=g)
                u = torch.where(torch.arange(u.shape[1], device=dev)[None, :] < thr[:, None], u, -1.0)
                v, i = torch.topk(u, min(K, u.shape[1]), dim=1)
                idx = torch.where(v >= 0, i, -1).to(torch.int32).contiguous()
            max_cmp = ncmp if mode == "hca" else 0
            slots = {"swa": 0, "hca": max_cmp, "csa": K}[mode]
            nws = lib.dsa_sparse_flash_mla_workspace_size(S, H, win, slots)
            ws = torch.empty((max(nws, 1),), dtype=torch.uint8, device=dev)

            def call():
                rc = lib.dsa_sparse_flash_mla(
                    L.KIND_BF16, q.data_ptr(), S, H, D, 1, qs.data_ptr(), ql.data_ptr(), kl.data_ptr(),
                    ori.data_ptr(), nb, bs, obt.data_ptr(), nb, L.ptr(cmp), 0 if cmp is None else cmp.shape[0], bs,
                    L.ptr(cbt), 0 if cbt is None else cbt.shape[1], L.ptr(idx), K, ratio, win, max_cmp,
                    sinks.data_ptr(), D ** -0.5, out.data_ptr(), lse.data_ptr(), ws.data_ptr(), nws,
                    L.stream_handle(dev))
                L.check(rc, "sparse_flash_mla")

            call()
            torch.cuda.synchronize()
            t = _timed_graph(torch, call, 20)
            keys = torch.clamp(sg, max=win) + 1
            if mode == "hca":
                keys = keys + thr
            elif mode == "csa":
                keys = keys + torch.clamp(thr, max=K)
            n_keys = int(keys.sum().item())
            flops = 4.0 * H * D * n_keys
            name = f"{mode}_{tag}"
            entry = {"us": round(t * 1e3, 2), "keys_per_row": round(n_keys / S, 1),
                     "reference_ascend_us": V4_REFERENCE_US[name],
                     "speedup_vs_reference": round(V4_REFERENCE_US[name] / (t * 1e3), 2)}
            if tag == "prefill":
                entry["tflops"] = round(flops / (t * 1e-3) / 1e12, 1)
                entry["frac_bf16_peak"] = round(flops / (t * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4)
            else:
                nbytes = n_keys * D * 2 + q.numel() * 2 + out.numel() * 2
                entry["gbs"] = round(nbytes / (t * 1e-3) / 1e9, 1)
            res[name] = entry
            _log(f"V4 {name}: {t * 1e3:.1f} us ({entry.get('tflops', entry.get('gbs'))})")
            del cmp, cbt, idx, ws
        del q, ori, obt, out, lse
    return res


# Published device times of the reference's sparse MLA (SFA) paged decode, TileLang and AscendC on
# Ascend A3 (examples/sparse_flash_attention/bench_sfa/README.md:31-34), per KV pool size.
SFA_REFERENCE_US = {2560: (109.760, 98.0), 6400: (109.100, 99.0), 48000: (108.980, 100.0)}


def run_gqa(torch, pkg, dev, args, flush):
    """The grouped 128-wide sparse attention at the shape of the reference's GQA example
    (examples/sparse_flash_attention/example_sparse_flash_attn_gqa.py:266-318): B=2, S=273,
    SKV=44444, 64 query heads over 4 KV heads, D=128 (K = V), topk 2048, fp16; every row draws
    2048 distinct positions below q_start = 28672.  No published figure: reported for its own
    bounds (the gathered rows, the unique HBM bytes, the MFMA work)."""
    from tilelang_ascend_amd import _lib as L
    lib = pkg.load_library()
    B, S, SKV, H, G, D, K, q_start = 2, 273, 44444, 64, 4, 128, 2048, 4096 * 7
    g = torch.Generator(device=dev).manual_seed(20261207)
    q = torch.randn((B, S, H, D), device=dev, generator=g).to(torch.float16)
    kv = torch.randn((B, SKV, G, D), device=dev, generator=g).to(torch.float16)
    idx = torch.rand((B * S * G, q_start), device=dev, generator=g).argsort(dim=1)[:, :K]
    idx = idx.to(torch.int32).view(B, S, G, K).contiguous()
    out = torch.empty((B, S, H, D), dtype=torch.float16, device=dev)
    lse = torch.empty((B, S, H), dtype=torch.float32, device=dev)
    stream = L.stream_handle(dev)

    def call():
        rc = lib.dsa_sparse_attention_fwd(L.KIND_FP16, q.data_ptr(), kv.data_ptr(), idx.data_ptr(), None, None, None,
                                          B, S, H, G, D, D, SKV, 0, 0, K, D ** -0.5, 1, out.data_ptr(),
                                          lse.data_ptr(), None, 0, stream)
        L.check(rc, "grouped sparse attention")

    call()
    torch.cuda.synchronize()
    t = _median(_timed(torch, call, args.reps, flush))
    gathered = B * S * G * K * D * 2
    unique = kv.numel() * 2 + q.numel() * 2 + out.numel() * 2 + lse.numel() * 4 + idx.numel() * 4
    flops = 4.0 * B * S * H * K * D
    res = {"workload": "GQA example shape: B=2, S=273, SKV=44444, H=64 over kv_group=4, D=128, topk=2048, fp16",
           "us": round(t * 1e3, 1),
           "gathered_bytes": gathered,
           "gather_gbs": round(gathered / (t * 1e-3) / 1e9, 1),
           "unique_hbm_bytes": unique,
           "hbm_floor_us": round(unique / (PEAK_HBM_GBS * 1e9) * 1e6, 1),
           "tflops": round(flops / (t * 1e-3) / 1e12, 1)}
    _log(f"GQA example shape: {t * 1e3:.1f} us, gathered rows {res['gather_gbs']:.0f} GB/s")
    del q, kv, idx, out, lse
    return res


def run_sfa_reference_shapes(torch, pkg, dev):
    """The reference's SFA decode benchmark (bench_sfa.py:9-70, :104-140): T=1, B=1, 128 heads,
    D=512 + 64 rope (one 576-wide latent row, V = its first 512), 2048 distinct indices drawn from
    act_kv=2560, 128-row blocks with an identity table, scale 0.5, sparse_mode 0, bf16; the KV
    pool holds 2560 / 6400 / 48000 rows.  Device time per call from a HIP graph, as the
    reference's figures are device task durations."""
    from tilelang_ascend_amd import _lib as L
    lib = pkg.load_library()
    g = torch.Generator(device=dev).manual_seed(20261206)
    H, D, bs, K, act = 128, 576, 128, 2048, 2560
    res = {"workload": "SFA paged decode of the reference benchmark: T=1, B=1, H=128, D=512+64, topk=2048 of "
                       "act_kv=2560, block 128, scale 0.5, sparse_mode 0, bf16; device time per call (HIP graph)"}
    q = (torch.randn((1, 1, H, D), device=dev, generator=g) * 0.5).to(torch.bfloat16)
    idx = torch.topk(torch.rand((1, act), device=dev, generator=g), K, dim=-1).indices.to(torch.int32)
    idx = idx.view(1, 1, 1, K).contiguous()
    kvl = torch.full((1,), act, dtype=torch.int32, device=dev)
    out = torch.empty((1, 1, H, 512), dtype=torch.bfloat16, device=dev)
    lse = torch.empty((1, 1, H), dtype=torch.float32, device=dev)
    nws = lib.dsa_sparse_mla_workspace_size(1, 1, H, K)
    ws = torch.empty((max(nws, 1),), dtype=torch.uint8, device=dev)
    for kv_s, (ref_tl, ref_ac) in SFA_REFERENCE_US.items():
        nb = kv_s // bs
        pool = (torch.randn((nb, bs, 1, D), device=dev, generator=g) * 0.5).to(torch.bfloat16)
        table = torch.arange(nb, dtype=torch.int32, device=dev).view(1, nb)

        def call():
            rc = lib.dsa_sparse_mla_fwd(L.KIND_BF16, q.data_ptr(), pool.data_ptr(), idx.data_ptr(), table.data_ptr(),
                                        None, kvl.data_ptr(), 1, 1, H, D, 512, nb * bs, bs, nb, K, 0.5, 0,
                                        out.data_ptr(), lse.data_ptr(), ws.data_ptr(), nws, L.stream_handle(dev))
            L.check(rc, "sfa decode")

        call()
        torch.cuda.synchronize()
        t = _timed_graph(torch, call, 20)
        res[f"kv_s_{kv_s}"] = {"us": round(t * 1e3, 2), "reference_tilelang_us": ref_tl, "reference_ascendc_us": ref_ac,
                               "speedup_vs_reference": round(ref_tl / (t * 1e3), 2)}
        _log(f"SFA decode KV_S={kv_s}: {t * 1e3:.1f} us (reference {ref_tl} us)")
        del pool, table
    return res


def _rocpd(db):
    import sqlite3

    return sqlite3.connect(f"file:{db}?mode=ro", uri=True)


def _kname(name):
    """Demangled kernel name without the return type and parameter list."""
    name = name.split("(")[0]
    return name[5:] if name.startswith("void ") else name


def summarize_trace(db, drop=0, label="", groups=1):
    """Per-kernel dispatch statistics from a `rocprofv3 --kernel-trace` rocpd database (durations in us).

    The first `drop` dispatches of every (kernel, grid) row are left out (the warmup launches of a
    bench part), so the averages cover the timed launches only; `label` names the workload.  With
    `groups` > 1 the remaining dispatches of a row are split into that many consecutive runs of equal
    length, one output row each (labelled #1, #2, ...), for a part that times one call several ways."""
    con = _rocpd(db)
    rows = con.execute("select name, grid_x * grid_y * grid_z, workgroup_x, duration, lds_size, scratch_size, "
                       "vgpr_count, accum_vgpr_count, start from kernels order by start").fetchall()
    agg = {}
    for name, grid, wg, dur, lds, scr, vg, ag, _start in rows:
        name = _kname(name)
        if not name.startswith("dsa::"):
            continue
        key = (name, grid, wg)
        agg.setdefault(key, {"d": [], "meta": (lds, scr, vg, ag)})["d"].append(dur / 1e3)
    print(f"{'workload':10s} {'kernel':48s} {'grid':>9s} {'wg':>4s} {'calls':>5s} {'avg_us':>10s} {'min_us':>10s} "
          f"{'max_us':>10s} lds/scratch/vgpr/agpr")
    for (name, grid, wg), v in sorted(agg.items(), key=lambda kv: -sum(kv[1]["d"])):
        d = v["d"][drop:] if len(v["d"]) > drop else v["d"]
        runs = [d]
        if groups > 1 and len(d) % groups == 0:
            n = len(d) // groups
            runs = [d[i * n:(i + 1) * n] for i in range(groups)]
        for i, r in enumerate(runs):
            tag = f"{label}#{i + 1}" if len(runs) > 1 else label
            print(f"{tag:10s} {name:48s} {grid:9d} {wg:4d} {len(r):5d} {sum(r) / len(r):10.1f} {min(r):10.1f} "
                  f"{max(r):10.1f} {'/'.join(str(x) for x in v['meta'])}")


def _counter_means(db, counter):
    """{(kernel, grid): mean KiB per dispatch} for one byte counter of a `rocprofv3 --pmc` database."""
    con = _rocpd(db)
    acc = {}
    for name, grid, cn, val in con.execute("select kernel_name, grid_size, counter_name, value "
                                           "from counters_collection"):
        if cn != counter:
            continue
        key = (_kname(name), grid)
        acc.setdefault(key, []).append(val)
    return {k: sum(v) / len(v) for k, v in acc.items()}


def summarize_traffic(fetch_db, write_db, cal_fetch_db, cal_write_db):
    """HBM bytes per dispatch of every dsa kernel: FETCH_SIZE and WRITE_SIZE scaled by a copy-kernel calibration.

    The calibration databases hold `bench.py --copy-calibration` (a 1 GiB device copy); the factor per
    counter is 1 GiB divided by what that counter reports for the copy kernel.
    """
    cal_bytes = float(1 << 30)
    fac = {}
    for cn, db in (("FETCH_SIZE", cal_fetch_db), ("WRITE_SIZE", cal_write_db)):
        copies = [v for (n, _g), v in _counter_means(db, cn).items() if n == COPY_KERNEL]
        if not copies:
            raise SystemExit(f"no {COPY_KERNEL} dispatch with {cn} in {db}")
        fac[cn] = cal_bytes / (copies[0] * 1024.0)
        print(f"calibration {cn}: copy of 1 GiB reads {copies[0]:.1f} KiB -> factor {fac[cn]:.4f}")
    fetch = _counter_means(fetch_db, "FETCH_SIZE")
    write = _counter_means(write_db, "WRITE_SIZE")
    print(f"{'kernel':42s} {'grid':>9s} {'FETCH_KiB':>14s} {'WRITE_KiB':>14s}  traffic_bytes")
    for key in sorted(set(fetch) & set(write)):
        if not key[0].startswith("dsa::"):
            continue
        tb = fetch[key] * 1024.0 * fac["FETCH_SIZE"] + write[key] * 1024.0 * fac["WRITE_SIZE"]
        print(f"{key[0]:42s} {key[1]:9d} {fetch[key]:14.1f} {write[key]:14.1f}  {tb:.4e}")


def summarize_mfma(util_db, mops_db):
    """MFMA evidence per dsa kernel: rocprofv3's MfmaUtil (MFMA-busy cycles over all SIMDs' active
    cycles, percent) and the FLOPs the hardware counted (SQ_INSTS_VALU_MFMA_MOPS_* x 512) per dispatch."""
    util = _counter_means(util_db, "MfmaUtil")
    mops = {cn: _counter_means(mops_db, cn) for cn in ("SQ_INSTS_VALU_MFMA_MOPS_BF16", "SQ_INSTS_VALU_MFMA_MOPS_F8",
                                                       "SQ_INSTS_VALU_MFMA_MOPS_F16")}
    print(f"{'kernel':48s} {'grid':>9s} {'MfmaUtil_%':>10s} {'bf16_FLOP':>11s} {'fp8_FLOP':>11s} {'f16_FLOP':>11s}")
    for key in sorted(util):
        if not key[0].startswith("dsa::"):
            continue
        f = [mops[cn].get(key, 0.0) * 512.0 for cn in mops]
        print(f"{key[0]:48s} {key[1]:9d} {util[key]:10.1f} {f[0]:11.4e} {f[1]:11.4e} {f[2]:11.4e}")


def profiled_traffic(kernel, grid):
    """HBM bytes per launch of (kernel, grid) from the committed counter summary, or None if it has none."""
    path = PROFILES / "traffic_c4_prefill_step.txt"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        parts = line.rsplit(None, 4)
        if len(parts) == 5 and parts[0].strip() == kernel and parts[1] == str(grid):
            return float(parts[4])
    return None


def main():
    if len(sys.argv) > 1 and sys.argv[1] in ("--rocprof-trace", "--rocprof-traffic", "--rocprof-mfma"):
        # Summaries of rocprofv3 databases written by profiling this script (no GPU needed).
        if sys.argv[1] == "--rocprof-trace":
            # --rocprof-trace DB [DROP [LABEL [GROUPS]]]
            summarize_trace(sys.argv[2], int(sys.argv[3]) if len(sys.argv) > 3 else 0,
                            sys.argv[4] if len(sys.argv) > 4 else "", int(sys.argv[5]) if len(sys.argv) > 5 else 1)
        elif sys.argv[1] == "--rocprof-mfma":
            summarize_mfma(*sys.argv[2:4])
        else:
            summarize_traffic(*sys.argv[2:6])
        return
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--reps", type=int, default=20, help="repetitions of the secondary (flushed) benchmarks")
    ap.add_argument("--skip", default="", help="comma list of parts to skip: step,indexer,decode,c5,v4,gqa,sfa,cpu")
    ap.add_argument("--only", default="", help="comma list of the only parts to run (the complement of --skip)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a 1 GiB device-to-device copy (HBM byte-counter calibration for rocprof)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); got --gpus {args.gpus}",
              file=sys.stderr)
        sys.exit(2)
    skip = set(filter(None, args.skip.split(",")))
    parts = {"step", "indexer", "decode", "c5", "v4", "gqa", "sfa", "cpu"}
    if args.only:
        skip |= parts - set(filter(None, args.only.split(",")))

    import torch
    import __graft_entry__

    pkg = __graft_entry__.load_package()
    pkg.load_library()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    if args.copy_calibration:
        src = torch.ones(1 << 28, dtype=torch.float32, device=dev)  # 1 GiB
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes_each_way": src.numel() * 4, "reps": 5}), flush=True)
        return

    # ---------------- step workload: sparse MLA prefill (C4) ----------------
    S, H, topk = 16384, 128, 2048
    sm_scale = 576 ** -0.5
    result = {}
    cpu_inputs = None
    flush = _flush_buffer(torch, dev)
    if "step" not in skip:
        result, cpu_inputs = run_step(torch, pkg, dev, args, S, H, topk, sm_scale, flush)


    # ---------------- indexer + top-k (C2) ----------------
    if "indexer" not in skip:
        _log("C2 indexer + top-k")
        qi, ki, wi, ksi = gen_indexer(torch, dev)
        S1, S2, Hi, K = qi.shape[1], ki.shape[1], qi.shape[2], 2048
        logits = torch.empty(1, S1, S2, dtype=torch.float32, device=dev)
        lib = pkg.load_library()
        from tilelang_ascend_amd import _lib as L

        stream = L.stream_handle(dev)
        out_idx = torch.empty(S1, K, dtype=torch.int32, device=dev)

        def run_logits():
            rc = lib.dsa_indexer_logits(L.KIND_FP8_E4M3, qi.data_ptr(), ki.data_ptr(), ksi.data_ptr(), wi.data_ptr(),
                                        1, S1, S2, Hi, 128, None, None, None, 0, 0, 3, logits.data_ptr(), S2, stream)
            L.check(rc, "indexer")

        def run_topk():
            rc = lib.dsa_topk_select(logits.data_ptr(), S2, S1, S2, K, None, 1, out_idx.data_ptr(), None, stream)
            L.check(rc, "topk")

        def run_both():
            run_logits()
            run_topk()

        fidx = torch.empty(S1, K, dtype=torch.int32, device=dev)
        fws_b = lib.dsa_lightning_indexer_fused_workspace_size(1, S1, S2, K)
        fws = torch.empty(fws_b, dtype=torch.uint8, device=dev)
        fcnt = torch.zeros(1, dtype=torch.int32, device=dev)

        def run_fused():
            rc = lib.dsa_lightning_indexer_fused(L.KIND_FP8_E4M3, qi.data_ptr(), ki.data_ptr(), ksi.data_ptr(),
                                                 wi.data_ptr(), 1, S1, S2, Hi, 128, None, None, None, 0, 0, 3, K,
                                                 fidx.data_ptr(), None, fws.data_ptr(), fws_b, stream)
            L.check(rc, "fused indexer")

        for f in (run_logits, run_topk, run_both, run_fused):
            f()
        L.check(lib.dsa_lightning_indexer_fused_fallback_rows(fws.data_ptr(), 1, S1, S2, K, fcnt.data_ptr(), stream),
                "fallback rows")
        torch.cuda.synchronize()
        fused_same = bool(torch.equal(fidx, out_idx))
        fused_fallback = int(fcnt.item())
        t_log = _median(_timed(torch, run_logits, args.reps, flush))
        t_topk = _median(_timed(torch, run_topk, args.reps, flush))
        t_both = _median(_timed(torch, run_both, args.reps, flush))
        t_fused = _median(_timed(torch, run_fused, args.reps, flush))
        causal_pairs = sum(min(S2, S2 - S1 + t + 1) for t in range(S1))
        idx_flops = 2.0 * Hi * 128 * S1 * S2
        idx_tflops = idx_flops / (t_log * 1e-3) / 1e12
        topk_bytes = S1 * S2 * 4 + S1 * K * 4
        topk_gbs = topk_bytes / (t_topk * 1e-3) / 1e9
        result["indexer_topk"] = {
            "workload": "C2: Sq=4096, Skv=32768, 64 heads x 128 fp8, per-token k scale, causal, top-2048",
            "us": round(t_both * 1e3, 1),
            "indexer_us": round(t_log * 1e3, 1),
            "topk_us": round(t_topk * 1e3, 1),
            "indexer_tflops_dense": round(idx_tflops, 1),
            "indexer_frac_fp8_peak": round(idx_tflops / PEAK_FP8_TFLOPS, 4),
            "indexer_causal_pair_frac": round(causal_pairs / (S1 * S2), 4),
            "topk_gbs": round(topk_gbs, 1),
            "topk_frac_hbm": round(topk_gbs / PEAK_HBM_GBS, 4),
            "roofline_us": round((idx_flops / (PEAK_FP8_TFLOPS * 1e12) + topk_bytes / (PEAK_HBM_GBS * 1e9)) * 1e6, 1),
            "fused_us": round(t_fused * 1e3, 1),
            "fused_frac_fp8_floor": round(idx_flops / (PEAK_FP8_TFLOPS * 1e12) * 1e6 / (t_fused * 1e3), 4),
            "fused_equals_dense": fused_same,
            "fused_fallback_rows": fused_fallback,
        }
        _log(f"C2: indexer {t_log * 1e3:.1f} us, topk {t_topk * 1e3:.1f} us, both {t_both * 1e3:.1f} us, "
             f"fused {t_fused * 1e3:.1f} us (same: {fused_same}, fallback rows {fused_fallback})")
        del qi, ki, wi, ksi, logits, out_idx, fidx, fws

    # ---------------- decode (C3) ----------------
    if "decode" not in skip:
        _log("C3 paged decode")
        qd, pool, table, idd, lens = gen_decode(torch, dev)
        B = qd.shape[0]
        from tilelang_ascend_amd import _lib as L

        lib = pkg.load_library()
        out_d = torch.empty(B, 1, H, 512, dtype=torch.bfloat16, device=dev)
        lse_d = torch.empty(B, 1, H, dtype=torch.float32, device=dev)
        ws_bytes = lib.dsa_sparse_mla_workspace_size(B, 1, H, topk)
        ws_d = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
        stream = L.stream_handle(dev)
        nblk = table.shape[1]
        bsz = pool.shape[1]

        def fnd():
            # The C ABI directly, on preallocated buffers: the timed region holds only the kernels.
            rc = lib.dsa_sparse_mla_fwd(L.KIND_BF16, qd.data_ptr(), pool.data_ptr(), idd.data_ptr(), table.data_ptr(),
                                        None, lens.data_ptr(), B, 1, H, 576, 512, nblk * bsz, bsz, nblk, topk,
                                        sm_scale, 1, out_d.data_ptr(), lse_d.data_ptr(), ws_d.data_ptr(), ws_bytes,
                                        stream)
            L.check(rc, "decode")

        fnd()
        torch.cuda.synchronize()
        t_dec = _median(_timed(torch, fnd, args.reps, flush))
        flush.zero_only = True
        t_dec_zero = _median(_timed(torch, fnd, args.reps, flush))
        flush.zero_only = False
        dec_bytes = (B * topk * 576 * 2 + qd.numel() * 2 + B * H * 512 * 2 + B * H * 4 + idd.numel() * 4
                     + table.numel() * 4)
        dec_gbs = dec_bytes / (t_dec * 1e-3) / 1e9
        dec_flops = 2.0 * B * H * topk * (576 + 512)
        result["decode"] = {
            "workload": "C3: B=64, Sq=1, H=128, topk=2048, 64K-token paged cache (64-token blocks)",
            "us": round(t_dec * 1e3, 1),
            "gbs": round(dec_gbs, 1),
            "frac_hbm": round(dec_gbs / PEAK_HBM_GBS, 4),
            "tflops": round(dec_flops / (t_dec * 1e-3) / 1e12, 1),
            "bytes": dec_bytes,
            "roofline_us": round(dec_bytes / (PEAK_HBM_GBS * 1e9) * 1e6, 1),
            # The reference's zero-fill flush alone: the fill's write-back then shares HBM with the call.
            "us_zero_fill_flush_only": round(t_dec_zero * 1e3, 1),
        }
        _log(f"C3 decode: {t_dec * 1e3:.1f} us, {dec_gbs:.0f} GB/s (zero-fill flush only: {t_dec_zero * 1e3:.1f} us)")
        del qd, pool, table, idd

    # ---------------- full DSA layer at 128K context (C5) ----------------
    if "c5" not in skip:
        result["layer_128k"] = run_c5(torch, pkg, dev, args, flush)

    # ---------------- V4 sparse flash MLA at the reference benchmark's shapes ----------------
    if "v4" not in skip:
        result["v4_sparse_flash_mla"] = run_v4(torch, pkg, dev, args, flush)

    # ---------------- the grouped 128-wide kernel at the reference's GQA example shape ----------------
    if "gqa" not in skip:
        result["gqa_example_shape"] = run_gqa(torch, pkg, dev, args, flush)

    # ---------------- the reference's own SFA decode benchmark shapes ----------------
    if "sfa" not in skip:
        result["sfa_decode_reference_shapes"] = run_sfa_reference_shapes(torch, pkg, dev)

    del flush
    if "cpu" not in skip and cpu_inputs is not None:
        _log("CPU baseline (oracle, bounded sample)")
        result["cpu_baseline"] = cpu_baseline_prefill(torch, *cpu_inputs)
        del cpu_inputs
        result["cpu_baselines_other"] = cpu_baselines_other(torch)
        result["cpu_model"] = _cpu_model()
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
