"""DeepSeek V4 sparse flash MLA on gfx950: window + compressed-KV attention with sinks.

Mirrors ``sparse_flash_mla(q, *, ori_kv, cmp_kv, cmp_sparse_indices, ...)`` of
``examples/deepseek_v4/sparse_flash_mla/sparse_flash_mla_api.py:94-253``: same
keywords, the same three scenarios (``swa``: window only; ``hca``: window plus
every compressed row below the causal threshold; ``csa``: window plus the
selected compressed rows), the same layouts (``TND`` / ``BSND`` queries, paged
``PA_ND`` caches) and the same return value (``out`` or ``(out, lse)``).  The
semantics are those of the golden, ``sparse_flash_mla_golden.py:55-160``.

Superset of the reference: any head count that is a multiple of 16 up to 1024
(the reference: N1 = 64).  Ascend tuning knobs (``core_num``) are accepted and
ignored.
"""
from __future__ import annotations

from typing import Optional, Tuple, Union

import torch

from . import _lib

D = 512
DEFAULT_CORE_NUM = 24  # accepted for signature compatibility; unused on gfx950

_KINDS = {torch.bfloat16: _lib.KIND_BF16, torch.float16: _lib.KIND_FP16}


def _paged(name: str, kv: torch.Tensor, table: torch.Tensor, B: int, dev) -> Tuple[torch.Tensor, torch.Tensor]:
    if kv.dim() != 4 or kv.shape[2] != 1 or kv.shape[3] != D:
        raise ValueError(f"{name} must be [block_num, block_size, 1, {D}], got {tuple(kv.shape)}")
    _lib.require_contiguous(name, kv)
    bt = table.to(device=dev, dtype=torch.int32).contiguous()
    if bt.dim() != 2 or bt.shape[0] != B:
        raise ValueError(f"{name} block table must be [B={B}, table_len], got {tuple(bt.shape)}")
    return kv, bt


def sparse_flash_mla(
    q: torch.Tensor,
    *,
    ori_kv: torch.Tensor,
    cmp_kv: Optional[torch.Tensor] = None,
    cmp_sparse_indices: Optional[torch.Tensor] = None,
    ori_block_table: torch.Tensor,
    cmp_block_table: Optional[torch.Tensor] = None,
    cu_seqlens_q: Optional[torch.Tensor] = None,
    seqused_q: Optional[torch.Tensor] = None,
    seqused_kv: torch.Tensor,
    sinks: torch.Tensor,
    softmax_scale: float,
    cmp_ratio: Optional[int] = None,
    ori_mask_mode: int = 4,
    cmp_mask_mode: int = 3,
    ori_win_left: int = 127,
    ori_win_right: int = 0,
    layout_q: str = "TND",
    layout_kv: str = "PA_ND",
    return_softmax_lse: bool = False,
    core_num: int = DEFAULT_CORE_NUM,
    topk_cmp: Optional[int] = None,
) -> Union[torch.Tensor, Tuple[torch.Tensor, torch.Tensor]]:
    """V4 attention; ``out`` [T, N1, 512] (TND) or [B, S, N1, 512] (BSND), and
    with ``return_softmax_lse`` also ``lse`` [T, N1] / [B, S, N1] fp32 (natural
    log, sink included).

    Argument checks follow sparse_flash_mla_api.py:117-123 and :195-196 (the
    reference's asserts raise ``AssertionError`` here too).
    """
    del seqused_q, core_num
    if ori_mask_mode != 4:
        raise AssertionError("only ori_mask_mode=4 supported")
    if not (cmp_mask_mode == 3 or cmp_kv is None):
        raise AssertionError("only cmp_mask_mode=3 supported")
    if ori_win_right != 0:
        raise AssertionError("only ori_win_right=0 supported")
    if layout_kv != "PA_ND":
        raise AssertionError("only layout_kv=PA_ND supported")
    if layout_q not in ("TND", "BSND"):
        raise AssertionError(f"unsupported layout_q={layout_q!r}")
    if q.dtype not in _KINDS:
        raise ValueError(f"unsupported torch dtype {q.dtype}")
    # Like the reference (:169-206), every other tensor is moved to q's device.
    dev = _lib.require_device(q)
    ori_kv = ori_kv.to(dev)
    cmp_kv = None if cmp_kv is None else cmp_kv.to(dev)
    if ori_kv.dtype != q.dtype or (cmp_kv is not None and cmp_kv.dtype != q.dtype):
        raise ValueError("ori_kv / cmp_kv must have the dtype of q")

    # Query rows: TND packs batches by cu_seqlens_q ([B+1], from 0); BSND pads
    # each batch to S (lengths from cu_seqlens_q when given) -- :135-166.
    if layout_q == "TND":
        if cu_seqlens_q is None:
            raise AssertionError("cu_seqlens_q is required for TND")
        if q.dim() != 3:
            raise ValueError(f"TND q must be [T, N1, D], got {tuple(q.shape)}")
        cu = torch.as_tensor(cu_seqlens_q).to(torch.int64).cpu().reshape(-1)
        B = cu.numel() - 1
        T, N1, Dq = q.shape
        q_start = cu[:-1]
        q_len = cu[1:] - cu[:-1]
        if B < 1 or int(cu[0]) < 0 or int(q_len.min()) < 0 or int(cu[-1]) > T:
            raise ValueError("cu_seqlens_q must be non-decreasing, start at >= 0 and end at <= T")
    else:
        if q.dim() != 4:
            raise ValueError(f"BSND q must be [B, S, N1, D], got {tuple(q.shape)}")
        B, S, N1, Dq = q.shape
        T = B * S
        q_start = torch.arange(B, dtype=torch.int64) * S
        q_len = torch.full((B,), S, dtype=torch.int64)
        if cu_seqlens_q is not None:
            cu = torch.as_tensor(cu_seqlens_q).to(torch.int64).cpu().reshape(-1)
            q_len = (cu[1:] - cu[:-1]).clamp(0, S)
    if ori_kv.dim() == 4:
        N2 = ori_kv.shape[2]
    else:
        N2 = -1
    if N1 % 16 != 0 or N1 > 1024 or N2 != 1 or Dq != D:
        raise ValueError(f"N1 must be a multiple of 16 (<= 1024), N2=1, D=512 (got N1={N1}, N2={N2}, D={Dq})")
    _lib.require_contiguous("q", q)
    kv_len = torch.as_tensor(seqused_kv).to(device=dev, dtype=torch.int32).reshape(-1).contiguous()
    if kv_len.numel() != B:
        raise ValueError(f"seqused_kv must have B={B} entries, got {kv_len.numel()}")
    ori, ori_bt = _paged("ori_kv", ori_kv, ori_block_table, B, dev)

    cmp, cmp_bt, idx = None, None, None
    K, max_cmp, ratio, cmp_slots = 0, 0, int(cmp_ratio) if cmp_ratio is not None else 4, 0
    if cmp_kv is not None:
        if cmp_block_table is None:
            raise ValueError("cmp_kv requires cmp_block_table")
        cmp, cmp_bt = _paged("cmp_kv", cmp_kv, cmp_block_table, B, dev)
        if cmp_sparse_indices is not None:
            ci = cmp_sparse_indices.to(device=dev, dtype=torch.int32)
            if layout_q == "BSND":
                ci = ci.reshape(T, ci.shape[2], ci.shape[3])
            if ci.dim() != 3 or ci.shape[0] != T or ci.shape[1] != 1:
                raise ValueError(f"cmp_sparse_indices must be [T, 1, K] (TND) or [B, S, 1, K], got "
                                 f"{tuple(cmp_sparse_indices.shape)}")
            K = topk_cmp if topk_cmp is not None else ci.shape[2]
            if ci.shape[2] != K:
                raise AssertionError("topk_cmp does not match cmp_sparse_indices last dim")
            idx = ci.reshape(T, K).contiguous()
            cmp_slots = K
        else:
            if cmp_ratio is None:
                raise ValueError("cmp_ratio is required with cmp_kv")
            max_cmp = int(kv_len.max().item()) // ratio
            cmp_slots = max_cmp
    sk = None if sinks is None else sinks.to(device=dev, dtype=torch.float32).reshape(-1).contiguous()
    if sk is not None and sk.numel() != N1:
        raise ValueError(f"sinks must hold one value per head ({N1}), got {sk.numel()}")

    out = torch.empty((T, N1, D), dtype=q.dtype, device=dev)
    lse = torch.empty((T, N1), dtype=torch.float32, device=dev)
    if T > 0:
        qs = q_start.to(device=dev, dtype=torch.int32).contiguous()
        ql = q_len.to(device=dev, dtype=torch.int32).contiguous()
        lib = _lib.load_library()
        ws_bytes = lib.dsa_sparse_flash_mla_workspace_size(T, N1, ori_win_left, cmp_slots)
        ws = torch.empty((max(ws_bytes, 1),), dtype=torch.uint8, device=dev)
        rc = lib.dsa_sparse_flash_mla(
            _KINDS[q.dtype], _lib.ptr(q), T, N1, D, B, _lib.ptr(qs), _lib.ptr(ql), _lib.ptr(kv_len),
            _lib.ptr(ori), ori.shape[0], ori.shape[1], _lib.ptr(ori_bt), ori_bt.shape[1],
            _lib.ptr(cmp), 0 if cmp is None else cmp.shape[0], 0 if cmp is None else cmp.shape[1], _lib.ptr(cmp_bt),
            0 if cmp_bt is None else cmp_bt.shape[1], _lib.ptr(idx), K, ratio, ori_win_left, max_cmp,
            _lib.ptr(sk), float(softmax_scale), _lib.ptr(out), _lib.ptr(lse), _lib.ptr(ws), ws_bytes,
            _lib.stream_handle(dev))
        _lib.check(rc, "dsa_sparse_flash_mla")
    if layout_q == "BSND":
        out = out.view(B, S, N1, D)
        lse = lse.view(B, S, N1)
    if return_softmax_lse:
        return out, lse
    return out


def sparse_attn(query_states: torch.Tensor, kv_states: torch.Tensor, attn_sink: torch.Tensor,
                topk_idxs: torch.Tensor, softmax_scale: float) -> torch.Tensor:
    """V4 gathered-index attention with sinks (examples/deepseek_v4/sparse_attention.py:171-198):
    q [b, m, h, 512], kv [b, n, 512], attn_sink [h] fp32, topk_idxs [b, m, topk] int32 (-1 =
    empty slot; duplicates count twice) -> fp32 [b, m, h, 512].  As the reference kernel
    (sparse_attention.py:56), the fp32 accumulator is written as it is: no 16-bit rounding."""
    if query_states.dtype not in _KINDS or kv_states.dtype != query_states.dtype:
        raise ValueError("query_states / kv_states must share a bfloat16 or float16 dtype")
    dev = _lib.require_device(query_states)
    if query_states.dim() != 4 or query_states.shape[-1] != D:
        raise ValueError(f"query_states must be [b, m, h, {D}], got {tuple(query_states.shape)}")
    b, m, h, _ = query_states.shape
    if kv_states.dim() != 3 or kv_states.shape[0] != b or kv_states.shape[2] != D:
        raise ValueError(f"kv_states must be [b, n, {D}], got {tuple(kv_states.shape)}")
    if h % 16 != 0 or h > 1024:
        raise ValueError(f"heads must be a multiple of 16 (<= 1024), got {h}")
    n = kv_states.shape[1]
    idx = topk_idxs.to(device=dev, dtype=torch.int32).contiguous()
    if idx.dim() != 3 or tuple(idx.shape[:2]) != (b, m):
        raise ValueError(f"topk_idxs must be [b, m, topk], got {tuple(topk_idxs.shape)}")
    topk = idx.shape[2]
    for name, t in (("query_states", query_states), ("kv_states", kv_states)):
        _lib.require_contiguous(name, t)
    kv = kv_states.to(dev)
    sk = None if attn_sink is None else attn_sink.to(device=dev, dtype=torch.float32).reshape(-1).contiguous()
    if sk is not None and sk.numel() != h:
        raise ValueError(f"attn_sink must hold one value per head ({h}), got {sk.numel()}")
    out = torch.empty((b, m, h, D), dtype=torch.float32, device=dev)
    lse = torch.empty((b, m, h), dtype=torch.float32, device=dev)
    if b * m > 0:
        lib = _lib.load_library()
        ws_bytes = lib.dsa_sparse_attn_sink_workspace_size(b, m, h, topk)
        ws = torch.empty((max(ws_bytes, 1),), dtype=torch.uint8, device=dev)
        rc = lib.dsa_sparse_attn_sink(_KINDS[query_states.dtype], _lib.ptr(query_states), _lib.ptr(kv),
                                      _lib.ptr(idx), b, m, h, n, D, topk, _lib.ptr(sk), float(softmax_scale),
                                      _lib.ptr(out), _lib.ptr(lse), _lib.ptr(ws), ws_bytes, _lib.stream_handle(dev))
        _lib.check(rc, "dsa_sparse_attn_sink")
    return out


def sparse_attn_kernel(h: int, d: int, scale: Optional[float] = None):
    """Builder with the signature of sparse_attention.py:28 (``sparse_attn_kernel(h, d, scale)``):
    returns ``kernel(q, kv, attn_sink, topk_idxs) -> fp32 [b, m, h, d]``; scale defaults to
    1/sqrt(d) as there."""
    if d != D:
        raise ValueError(f"d must be {D}, got {d}")
    sc = (1.0 / d) ** 0.5 if scale is None else scale

    def kernel(q: torch.Tensor, kv: torch.Tensor, attn_sink: torch.Tensor, topk_idxs: torch.Tensor) -> torch.Tensor:
        if q.shape[2] != h:
            raise ValueError(f"q must have {h} heads, got {q.shape[2]}")
        return sparse_attn(q, kv, attn_sink, topk_idxs, sc)

    return kernel
