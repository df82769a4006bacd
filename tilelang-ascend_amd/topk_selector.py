"""Top-k selector (``examples/topk_selector/example_topk_selector.py``), gfx950 radix select.

``topk_selector(x, top_k)`` and the builder ``simple_topk_selector(B, N, top_k,
block_N)`` (reference signature, example_topk_selector.py:19) return int32
indices of the ``top_k`` largest scores per row, ordered (value desc, index asc)
-- the stable rule of examples/deepseek_v4/lightning_indexer.py:317-325 rather
than ``torch.topk``'s unspecified tie order.  Scores <= -1e30 (and -inf, NaN)
never take a slot; unfilled slots hold -1.
"""
from __future__ import annotations

from typing import Optional, Tuple, Union

import torch

from . import _lib


def topk_selector(x: torch.Tensor, top_k: int, sorted: bool = True, *, row_len: Optional[torch.Tensor] = None,
                  return_values: bool = False) -> Union[torch.Tensor, Tuple[torch.Tensor, torch.Tensor]]:
    """Row-wise top-k over the last dimension of ``x`` ([..., N]).

    Returns int32 indices [..., top_k] (and fp32 values if ``return_values``).
    ``row_len`` (int32, one per row) excludes columns >= row_len[r].
    fp16/bf16 inputs are widened to fp32 on the device (exact).
    """
    if x.dim() < 1:
        raise ValueError("x must have at least one dimension")
    if not (1 <= top_k <= 8192):
        raise ValueError(f"top_k must be in [1, 8192], got {top_k}")
    if x.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        raise ValueError(f"x must be float32/float16/bfloat16, got {x.dtype}")
    dev = _lib.require_device(x, row_len)
    lead = x.shape[:-1]
    n = x.shape[-1]
    xf = x.float() if x.dtype != torch.float32 else x
    xf = xf.reshape(-1, n)
    if xf.stride(-1) != 1 or (xf.shape[0] > 1 and xf.stride(0) < n):
        xf = xf.contiguous()
    rows = xf.shape[0]
    ld = xf.stride(0) if rows > 1 else n
    if row_len is not None:
        if row_len.numel() != rows:
            raise ValueError(f"row_len must have one entry per row ({rows}), got {row_len.numel()}")
        row_len = row_len.to(torch.int32).contiguous()
    idx = torch.empty((rows, top_k), dtype=torch.int32, device=dev)
    val = torch.empty((rows, top_k), dtype=torch.float32, device=dev) if return_values else None
    lib = _lib.load_library()
    ws_bytes = lib.dsa_topk_select_workspace_size(rows, n, top_k)
    ws = torch.empty((ws_bytes,), dtype=torch.uint8, device=dev) if ws_bytes else None
    rc = lib.dsa_topk_select_ws(_lib.ptr(xf), ld, rows, n, top_k, _lib.ptr(row_len), 1 if sorted else 0,
                                _lib.ptr(idx), _lib.ptr(val), _lib.ptr(ws), ws_bytes, _lib.stream_handle(dev))
    _lib.check(rc, "dsa_topk_select_ws")
    idx = idx.view(*lead, top_k)
    if return_values:
        return idx, val.view(*lead, top_k)
    return idx


def simple_topk_selector(B: int, N: int, top_k: int, block_N: Optional[int] = None, dtype: str = "float32"):
    """Builder with the reference's signature (example_topk_selector.py:19): returns ``kernel(x) -> indices``.

    ``block_N`` (the reference's UB chunk) has no meaning here and is ignored.
    """
    if dtype != "float32":
        raise ValueError(f"dtype must be float32, got {dtype}")

    def kernel(x: torch.Tensor) -> torch.Tensor:
        if tuple(x.shape) != (B, N):
            raise ValueError(f"expected x of shape {(B, N)}, got {tuple(x.shape)}")
        if x.dtype != torch.float32:
            raise ValueError(f"expected float32 x, got {x.dtype}")
        return topk_selector(x, top_k, sorted=True)

    return kernel
