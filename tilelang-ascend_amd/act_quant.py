"""Per-row activation quantiser on gfx950: the producer of the indexer's low-precision inputs.

``act_quant(x, round_scale=False, dtype=torch.int8)`` mirrors ``act_quant_torch``
(examples/deepseek_v4/act_quant.py:118-142) and the kernel it checks,
``act_quant_kernel_int8_optimized`` (:33-92): per row, scale = max(|x|, 1e-4) /
127 (or its power-of-two ceiling with ``round_scale``), y = round-half-even of
clamp(x / scale, -127, 127) as int8.  ``dtype=torch.float8_e4m3fn`` applies the
same recipe with 448 and a round-to-nearest-even conversion to OCP e4m3fn --
the input format of the fp8 lightning indexer (keys with their per-row scale as
``key_scale``; a query's per-(token, head) scale folds into the head weights,
``lightning_indexer(..., query_scale=...)``).
"""
from __future__ import annotations

from typing import Tuple

import torch

from . import _lib

_IN = {torch.bfloat16: _lib.KIND_BF16, torch.float16: _lib.KIND_FP16, torch.float32: _lib.KIND_FP32}
_OUT = {torch.int8: _lib.KIND_INT8, torch.float8_e4m3fn: _lib.KIND_FP8_E4M3}


def act_quant(x: torch.Tensor, round_scale: bool = False,
              dtype: torch.dtype = torch.int8) -> Tuple[torch.Tensor, torch.Tensor]:
    """(y, scales): y has x's shape in ``dtype``; scales [M, 1] fp32 for a 2-D x
    ([B, S, 1] for a 3-D one, as act_quant.py:138-140 returns them)."""
    if x.dtype not in _IN:
        raise ValueError(f"x must be bfloat16, float16 or float32, got {x.dtype}")
    if dtype not in _OUT:
        raise ValueError(f"dtype must be torch.int8 or torch.float8_e4m3fn, got {dtype}")
    if x.dim() not in (2, 3):
        raise ValueError(f"x must be [M, N] or [B, S, N], got {tuple(x.shape)}")
    dev = _lib.require_device(x)
    _lib.require_contiguous("x", x)
    n = x.shape[-1]
    rows = x.numel() // n if n else 0
    y = torch.empty(x.shape, dtype=dtype, device=dev)
    scales = torch.empty(x.shape[:-1] + (1,), dtype=torch.float32, device=dev)
    if rows and n:
        rc = _lib.load_library().dsa_act_quant(_IN[x.dtype], _lib.ptr(x), rows, n, _OUT[dtype], _lib.ptr(y),
                                               _lib.ptr(scales), 1 if round_scale else 0, _lib.stream_handle(dev))
        _lib.check(rc, "dsa_act_quant")
    return y, scales
