"""Lightning indexer on gfx950: fp8/bf16/fp16 MFMA logits, then the radix top-k.

Mirrors the host interface of ``examples/deepseek_v4/lightning_indexer.py:1202-1370``
(``lightning_indexer(query, key, weights, *, actual_seq_lengths_query, ...)``
returning ``(indices [B, S1, 1, K] int32, values)``) and the builder
``indexer(B, N2, G, S1, S2, D, TOP_K, ...)`` of
``examples/lightning_indexer/example_lightning_indexer.py:19-20``.

Superset of the reference: fp8-e4m3 (``torch.float8_e4m3fn``) query/key with an
optional per-key fp32 scale (``key_scale``); the logit is
``key_scale[s] * sum_h w[t, h] * ReLU(q[t, h] . k[s])``.  With fp16/bf16 inputs
and no scale it is the reference formula.  A quantised query's per-(token,
head) scale (``query_scale``, from ``act_quant``) is folded into the head
weights: ReLU(s x) = s ReLU(x) for s >= 0.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import _lib

_INT64_MAX = (1 << 63) - 1

_KINDS = {
    torch.float8_e4m3fn: _lib.KIND_FP8_E4M3,
    torch.bfloat16: _lib.KIND_BF16,
    torch.float16: _lib.KIND_FP16,
}


def _per_batch(seq_len: Optional[torch.Tensor], B: int, default: int, device) -> Optional[torch.Tensor]:
    if seq_len is None:
        return None
    t = torch.as_tensor(seq_len).to(device=device, dtype=torch.int32).reshape(-1).contiguous()
    if t.numel() != B:
        raise ValueError(f"actual sequence lengths must have B={B} entries, got {t.numel()}")
    return t


def _check_common(query, key, weights, layout_query, layout_key, sparse_mode):
    if layout_query not in ("BSND", "TND"):
        raise ValueError(f"Unsupported query layout: {layout_query}")
    if layout_key not in ("BSND", "PA_BSND", "TND"):
        raise ValueError(f"Unsupported key layout: {layout_key}")
    if layout_key != "PA_BSND" and layout_query != layout_key:
        raise ValueError(f"layout_query({layout_query}) must equal layout_key({layout_key}) when key is non-PA_BSND")
    if sparse_mode not in (0, 3):
        raise ValueError(f"sparse_mode must be 0 (defaultMask) or 3 (rightDownCausal), got {sparse_mode}")
    if query.dtype != key.dtype:
        raise ValueError(f"query dtype {query.dtype} must equal key dtype {key.dtype}")
    if query.dtype not in _KINDS:
        raise ValueError(f"query/key dtype must be float16, bfloat16 or float8_e4m3fn, got {query.dtype}")
    if weights.dtype not in (torch.float32, query.dtype) and not (query.dtype == torch.float8_e4m3fn):
        raise ValueError(f"weights dtype {weights.dtype} must be float32 or same as query {query.dtype}")


def _check_heads(N1, D):
    if D not in (64, 128):
        raise ValueError(f"head dim must be 64 or 128, got {D}")
    if N1 > 64 or N1 < 1:
        raise ValueError(f"query head_num (N1) must be <= 64, got {N1}")


def _paged_key(key, block_table, actual_seq_lengths_key, B, D, dev):
    """PA_BSND key: (block_table, block_size, max_blocks, per-batch lengths, S2)."""
    if block_table is None:
        raise ValueError("PA_BSND layout requires block_table")
    if actual_seq_lengths_key is None:
        raise ValueError("PA_BSND case requires actual_seq_lengths_key")
    if key.dim() != 4 or key.shape[2] != 1 or key.shape[3] != D:
        raise ValueError(f"PA_BSND key must be [blocks, block_size, 1, {D}], got {tuple(key.shape)}")
    block_size = key.shape[1]
    if block_size % 16 != 0 or block_size > 1024 or block_size <= 0:
        raise ValueError(f"PA block_size must be a positive multiple of 16 and <= 1024, got {block_size}")
    bt = block_table.to(torch.int32).contiguous()
    if bt.dim() != 2 or bt.shape[0] != B:
        raise ValueError(f"block_table must be [B, max_blocks], got {tuple(bt.shape)}")
    max_blocks = bt.shape[1]
    ak = _per_batch(actual_seq_lengths_key, B, 0, dev)
    S2 = int(ak.max().item()) if B > 0 else 0
    if S2 > max_blocks * block_size:
        raise ValueError("actual_seq_lengths_key exceeds block_table capacity")
    return bt, block_size, max_blocks, ak, S2


def _fold_query_scale(w, query_scale):
    """Head weights times the query's per-(token, head) scale (non-negative)."""
    if query_scale is None:
        return w
    qs = query_scale.to(device=w.device, dtype=torch.float32)
    if qs.numel() != w.numel():
        raise ValueError(f"query_scale must hold one fp32 per (token, head) ({w.numel()}), got {qs.numel()}")
    return (w * qs.reshape(w.shape)).contiguous()


def _key_scale(key_scale, rows):
    if key_scale is None:
        return None
    ks = key_scale.to(torch.float32).contiguous()
    if ks.numel() != rows:
        raise ValueError(f"key_scale must hold one fp32 per key row ({rows}), got {ks.numel()}")
    return ks


def _prefix_sums(seq, total, what, dev):
    """Inclusive prefix sums of a TND layout: int32 [B] on ``dev`` and the
    per-batch lengths on the host (lightning_indexer.py:68-71, :136-138)."""
    if seq is None:
        raise ValueError(f"TND layout requires {what} (prefix sums)")
    cu = torch.as_tensor(seq).reshape(-1).to(dtype=torch.int64)
    host = cu.cpu()
    if host.numel() == 0:
        raise ValueError(f"{what} must have at least one batch")
    lens = torch.diff(host, prepend=host.new_zeros(1))
    if int(lens.min()) < 0:
        raise ValueError(f"{what} must be non-decreasing prefix sums starting at >= 0")
    if int(host[-1]) > total:
        raise ValueError(f"{what} ends at {int(host[-1])}, beyond the {total} packed rows")
    return cu.to(device=dev, dtype=torch.int32).contiguous(), lens


def _prepare_tnd(query, key, weights, key_scale, actual_seq_lengths_query, actual_seq_lengths_key, block_table,
                 layout_key, query_scale=None):
    """Packed query rows [T, N1, D] addressed in place through prefix sums
    (the reference pads them to BSND on the host, lightning_indexer.py:48-94)."""
    dev = _lib.require_device(query, key, weights, key_scale, block_table)
    if query.dim() != 3:
        raise ValueError(f"TND query must be [T, N1, D], got {tuple(query.shape)}")
    T, N1, D = query.shape
    _check_heads(N1, D)
    cu_q, q_lens = _prefix_sums(actual_seq_lengths_query, T, "actual_seq_lengths_query", dev)
    B = cu_q.numel()
    S1 = int(q_lens.max())
    cu_k = ak = bt = None
    block_size = max_blocks = 0
    if layout_key == "PA_BSND":
        bt, block_size, max_blocks, ak, S2 = _paged_key(key, block_table, actual_seq_lengths_key, B, D, dev)
        ks = _key_scale(key_scale, key.shape[0] * key.shape[1])
    else:
        if key.dim() != 3 or key.shape[1] != 1 or key.shape[2] != D:
            raise ValueError(f"TND key must be [T_k, 1, {D}] (N2 = 1), got {tuple(key.shape)}")
        cu_k, k_lens = _prefix_sums(actual_seq_lengths_key, key.shape[0], "actual_seq_lengths_key", dev)
        if cu_k.numel() != B:
            raise ValueError(f"actual_seq_lengths_key must have B={B} entries, got {cu_k.numel()}")
        S2 = int(k_lens.max())
        ks = _key_scale(key_scale, key.shape[0])
    if tuple(weights.shape[:2]) != (T, N1) or weights.numel() != T * N1:
        raise ValueError(f"TND weights must be [T, N1] = {(T, N1)}, got {tuple(weights.shape)}")
    for name, t in (("query", query), ("key", key)):
        _lib.require_contiguous(name, t)
    w = _fold_query_scale(weights.reshape(T, N1).to(torch.float32).contiguous(), query_scale)
    T_rows = int(cu_q[-1].item())
    return dev, B, T, T_rows, S1, S2, N1, D, w, ks, cu_q, cu_k, ak, bt, block_size, max_blocks


def _prepare(query, key, weights, key_scale, actual_seq_lengths_query, actual_seq_lengths_key, block_table,
             layout_query, layout_key, sparse_mode, query_scale=None):
    _check_common(query, key, weights, layout_query, layout_key, sparse_mode)
    dev = _lib.require_device(query, key, weights, key_scale, block_table)
    if query.dim() != 4:
        raise ValueError(f"BSND query must be [B, S1, N1, D], got {tuple(query.shape)}")
    B, S1, N1, D = query.shape
    _check_heads(N1, D)
    is_pa = layout_key == "PA_BSND"
    if is_pa:
        bt, block_size, max_blocks, ak, S2 = _paged_key(key, block_table, actual_seq_lengths_key, B, D, dev)
    else:
        if key.dim() != 4 or key.shape[0] != B or key.shape[2] != 1 or key.shape[3] != D:
            raise ValueError(f"BSND key must be [B, S2, 1, {D}] (N2 = 1), got {tuple(key.shape)}")
        S2 = key.shape[1]
        bt, block_size, max_blocks = None, 0, 0
        ak = _per_batch(actual_seq_lengths_key, B, S2, dev)
        if ak is not None and B > 0 and int(ak.max().item()) > S2:
            raise ValueError("actual_seq_lengths_key exceeds the key's S2")
    aq = _per_batch(actual_seq_lengths_query, B, S1, dev)
    if aq is not None and B > 0 and int(aq.max().item()) > S1:
        raise ValueError("actual_seq_lengths_query exceeds the query's S1")
    if tuple(weights.shape[:3]) != (B, S1, N1) or weights.numel() != B * S1 * N1:
        raise ValueError(f"weights must be [B, S1, N1] = {(B, S1, N1)}, got {tuple(weights.shape)}")
    for name, t in (("query", query), ("key", key)):
        _lib.require_contiguous(name, t)
    w = _fold_query_scale(weights.reshape(B, S1, N1).to(torch.float32).contiguous(), query_scale)
    ks = _key_scale(key_scale, key.shape[0] * key.shape[1])
    return dev, B, S1, S2, N1, D, w, ks, aq, ak, bt, block_size, max_blocks


def indexer_logits(query: torch.Tensor, key: torch.Tensor, weights: torch.Tensor,
                   key_scale: Optional[torch.Tensor] = None, *,
                   actual_seq_lengths_query: Optional[torch.Tensor] = None,
                   actual_seq_lengths_key: Optional[torch.Tensor] = None,
                   block_table: Optional[torch.Tensor] = None, layout_query: str = "BSND",
                   layout_key: str = "BSND", sparse_mode: int = 3,
                   query_scale: Optional[torch.Tensor] = None) -> torch.Tensor:
    """fp32 logits [B, S1, S2] (masked positions -inf), the scores the top-k stage ranks.

    With ``layout_query="TND"`` the logits are [T, S2_max], one row per packed
    query row (S2_max = the longest key length of the batch)."""
    if layout_query == "TND":
        _check_common(query, key, weights, layout_query, layout_key, sparse_mode)
        (dev, B, T, T_rows, S1, S2, N1, D, w, ks, cu_q, cu_k, ak, bt, bs,
         mb) = _prepare_tnd(query, key, weights, key_scale, actual_seq_lengths_query, actual_seq_lengths_key,
                            block_table, layout_key, query_scale)
        out = torch.full((T_rows, S2), float("-inf"), dtype=torch.float32, device=dev)
        if T_rows == 0 or S2 == 0:
            return out
        lib = _lib.load_library()
        rc = lib.dsa_indexer_logits_tnd(_KINDS[query.dtype], _lib.ptr(query), _lib.ptr(key), _lib.ptr(ks),
                                        _lib.ptr(w), B, T_rows, S1, S2, N1, D, _lib.ptr(cu_q), _lib.ptr(cu_k),
                                        _lib.ptr(ak), _lib.ptr(bt), bs, mb, sparse_mode, _lib.ptr(out), S2,
                                        _lib.stream_handle(dev))
        _lib.check(rc, "dsa_indexer_logits_tnd")
        return out
    dev, B, S1, S2, N1, D, w, ks, aq, ak, bt, bs, mb = _prepare(
        query, key, weights, key_scale, actual_seq_lengths_query, actual_seq_lengths_key, block_table,
        layout_query, layout_key, sparse_mode, query_scale)
    out = torch.empty((B, S1, S2), dtype=torch.float32, device=dev)
    lib = _lib.load_library()
    rc = lib.dsa_indexer_logits(_KINDS[query.dtype], _lib.ptr(query), _lib.ptr(key), _lib.ptr(ks), _lib.ptr(w),
                                B, S1, S2, N1, D, _lib.ptr(aq), _lib.ptr(ak), _lib.ptr(bt), bs, mb, sparse_mode,
                                _lib.ptr(out), S2, _lib.stream_handle(dev))
    _lib.check(rc, "dsa_indexer_logits")
    return out


def lightning_indexer(query: torch.Tensor, key: torch.Tensor, weights: torch.Tensor, *,
                      actual_seq_lengths_query: Optional[torch.Tensor] = None,
                      actual_seq_lengths_key: Optional[torch.Tensor] = None,
                      block_table: Optional[torch.Tensor] = None, layout_query: str = "BSND",
                      layout_key: str = "BSND", sparse_count: int = 2048, sparse_mode: int = 3,
                      pre_tokens: int = _INT64_MAX, next_tokens: int = _INT64_MAX, return_value: bool = False,
                      key_scale: Optional[torch.Tensor] = None, query_scale: Optional[torch.Tensor] = None,
                      fuse_topk: Optional[bool] = None, **tuning) -> Tuple[torch.Tensor, torch.Tensor]:
    """Top-``sparse_count`` key positions per query row: (indices [B, S1, 1, K] int32, values).

    Validation follows lightning_indexer.py:1229-1257.  ``layout_query="TND"``
    takes packed query rows [T, N1, D] and weights [T, N1] with
    ``actual_seq_lengths_query`` as prefix sums, keys either packed
    (``layout_key="TND"``, [T_k, 1, D], prefix sums) or paged (``"PA_BSND"``,
    per-batch lengths), and returns [T', 1, K] with T' the last prefix sum
    (T on the empty early exit, lightning_indexer.py:1289-1296).  ``values`` is
    [B, S1, 1, K] (query dtype; fp32 for fp8 inputs) when ``return_value``, else
    an empty tensor.  Ascend tuning knobs (``block_n``, ``pp_slots``,
    ``max_cores``) are accepted and ignored.  ``fuse_topk`` streams
    the top-k out of the indexer without writing every row's logits, where the
    shape allows (``dsa_lightning_indexer_fused``); the output is the same bit for
    bit.  The default (None) streams calls of at least 2048 rows longer than 32768 keys, where it
    is faster.
    """
    unknown = set(tuning) - {"block_n", "pp_slots", "max_cores"}
    if unknown:
        raise TypeError(f"unexpected keyword arguments {sorted(unknown)}")
    if layout_key == "PA_BSND" and return_value:
        raise ValueError("PA_BSND layout does not support return_value")
    if not (1 <= sparse_count <= 2048 or (sparse_count % 1024 == 0 and sparse_count <= 8192)):
        raise ValueError(f"sparse_count must be in [1,2048] or a multiple of 1024 up to 8192, got {sparse_count}")
    if pre_tokens != _INT64_MAX:
        raise ValueError(f"pre_tokens must be INT64_MAX, got {pre_tokens}")
    if next_tokens != _INT64_MAX:
        raise ValueError(f"next_tokens must be INT64_MAX, got {next_tokens}")
    if layout_query == "TND":
        return _lightning_indexer_tnd(query, key, weights, key_scale, actual_seq_lengths_query,
                                      actual_seq_lengths_key, block_table, layout_key, sparse_count, sparse_mode,
                                      return_value, query_scale, fuse_topk)
    dev, B, S1, S2, N1, D, w, ks, aq, ak, bt, bs, mb = _prepare(
        query, key, weights, key_scale, actual_seq_lengths_query, actual_seq_lengths_key, block_table,
        layout_query, layout_key, sparse_mode, query_scale)
    idx = torch.empty((B, S1, 1, sparse_count), dtype=torch.int32, device=dev)
    vdt = torch.float32 if query.dtype == torch.float8_e4m3fn else query.dtype
    if B * S1 == 0 or S2 == 0:
        idx.fill_(-1)
        vals = (torch.full((B, S1, 1, sparse_count), float("-inf"), dtype=vdt, device=dev) if return_value
                else torch.empty((0,), dtype=vdt, device=dev))
        return idx, vals
    val = torch.empty((B, S1, 1, sparse_count), dtype=torch.float32, device=dev) if return_value else None
    lib = _lib.load_library()
    if fuse_topk is None:
        fuse_topk = _fuse_by_default(B * S1, S2)
    name = "dsa_lightning_indexer_fused" if fuse_topk else "dsa_lightning_indexer"
    ws_bytes = getattr(lib, name + "_workspace_size")(B, S1, S2, sparse_count)
    ws = torch.empty((ws_bytes,), dtype=torch.uint8, device=dev)
    rc = getattr(lib, name)(_KINDS[query.dtype], _lib.ptr(query), _lib.ptr(key), _lib.ptr(ks), _lib.ptr(w),
                            B, S1, S2, N1, D, _lib.ptr(aq), _lib.ptr(ak), _lib.ptr(bt), bs, mb, sparse_mode,
                            sparse_count, _lib.ptr(idx), _lib.ptr(val), _lib.ptr(ws), ws_bytes,
                            _lib.stream_handle(dev))
    _lib.check(rc, name)
    if return_value:
        return idx, val.to(vdt)
    return idx, torch.empty((0,), dtype=vdt, device=dev)


def _fuse_by_default(rows: int, S2: int) -> bool:
    """The streamed top-k pays off for long rows (over 32768 keys, where the dense top-k takes two
    stages) when there are enough of them (2048) for its launch to keep the dense pass's key chunks."""
    return S2 > 32768 and rows >= 2048


def _lightning_indexer_tnd(query, key, weights, key_scale, actual_seq_lengths_query, actual_seq_lengths_key,
                           block_table, layout_key, sparse_count, sparse_mode, return_value, query_scale=None,
                           fuse_topk=None):
    _check_common(query, key, weights, "TND", layout_key, sparse_mode)
    (dev, B, T, T_rows, S1, S2, N1, D, w, ks, cu_q, cu_k, ak, bt, bs,
     mb) = _prepare_tnd(query, key, weights, key_scale, actual_seq_lengths_query, actual_seq_lengths_key,
                        block_table, layout_key, query_scale)
    vdt = torch.float32 if query.dtype == torch.float8_e4m3fn else query.dtype
    if S1 == 0 or S2 == 0:
        idx = torch.full((T, 1, sparse_count), -1, dtype=torch.int32, device=dev)
        vals = (torch.full((T, 1, sparse_count), float("-inf"), dtype=vdt, device=dev) if return_value
                else torch.empty((0,), dtype=vdt, device=dev))
        return idx, vals
    idx = torch.empty((T_rows, 1, sparse_count), dtype=torch.int32, device=dev)
    val = torch.empty((T_rows, 1, sparse_count), dtype=torch.float32, device=dev) if return_value else None
    lib = _lib.load_library()
    if fuse_topk is None:
        fuse_topk = _fuse_by_default(T_rows, S2)
    if fuse_topk:
        name = "dsa_lightning_indexer_tnd_fused"
        ws_bytes = lib.dsa_lightning_indexer_tnd_fused_workspace_size(B, T_rows, S1, S2, sparse_count)
    else:
        name = "dsa_lightning_indexer_tnd"
        ws_bytes = lib.dsa_lightning_indexer_tnd_workspace_size(T_rows, S2, sparse_count)
    ws = torch.empty((ws_bytes,), dtype=torch.uint8, device=dev)
    rc = getattr(lib, name)(_KINDS[query.dtype], _lib.ptr(query), _lib.ptr(key), _lib.ptr(ks),
                            _lib.ptr(w), B, T_rows, S1, S2, N1, D, _lib.ptr(cu_q), _lib.ptr(cu_k),
                            _lib.ptr(ak), _lib.ptr(bt), bs, mb, sparse_mode, sparse_count, _lib.ptr(idx),
                            _lib.ptr(val), _lib.ptr(ws), ws_bytes, _lib.stream_handle(dev))
    _lib.check(rc, name)
    if return_value:
        return idx, val.to(vdt)
    return idx, torch.empty((0,), dtype=vdt, device=dev)


def indexer(B: int, N2: int, G: int, S1: int, S2: int, D: int, TOP_K: int, VECTOR_BASEN: int = 0,
            VECTOR_BASEG: int = 0, BLOCK_M: int = 0, BLOCK_N: int = 0, BLOCK_K: int = 0,
            input_dtype: str = "float16", calc_dtype: str = "float"):
    """Builder with the signature of example_lightning_indexer.py:19-20.

    Returns ``kernel(q [B, S1, N2, G*D], k [B, S2, N2, D], weights [B, S1, N2, G, 1])
    -> int32 [B, N2, S1, TOP_K]``: no causal mask, ranked by the head-weighted
    ReLU scores (example_lightning_indexer.py:137-144).  Tile arguments are
    Ascend tuning knobs and are ignored.  N2 must be 1.
    """
    if N2 != 1:
        raise ValueError(f"N2 must be 1, got {N2}")
    want = {"float16": torch.float16, "bfloat16": torch.bfloat16, "float8_e4m3fn": torch.float8_e4m3fn}
    if input_dtype not in want:
        raise ValueError(f"unsupported input_dtype {input_dtype}")

    def kernel(q: torch.Tensor, k: torch.Tensor, weights: torch.Tensor) -> torch.Tensor:
        if q.dtype != want[input_dtype] or k.dtype != want[input_dtype]:
            raise ValueError(f"q and k must be {input_dtype}")
        qb = q.reshape(B, S1, G, D).contiguous()
        kb = k.reshape(B, S2, 1, D).contiguous()
        wb = weights.reshape(B, S1, G)
        idx, _ = lightning_indexer(qb, kb, wb, sparse_count=TOP_K, sparse_mode=0)
        return idx.view(B, S1, 1, TOP_K).permute(0, 2, 1, 3).contiguous()

    return kernel
