"""Sparse MLA forward on gfx950: gathered latent-KV attention with LSE.

``sparse_mla_fwd(q, kv, indices, sm_scale)`` returns ``(out, lse)``:

* q       [B, S, H, 576] bf16/fp16 (512 latent + 64 rope dims)
* kv      [B, Skv, G, 576] (G latent KV heads, usually one), or a paged pool
          [num_blocks, block_size, G, 576] with ``block_table`` [B, max_blocks]
* indices [B, S, G, topk] int32 (or [B, S, topk] for G = 1), -1 = empty slot
* out     [B, S, H, 512] (V = kv[..., :512]), lse [B, S, H] fp32, natural log

With G > 1 query heads g*H/G .. (g+1)*H/G - 1 read KV head g through
indices[:, :, g] (the builder's ``kv_group``).  ``sparse_gqa_fwd`` is the same
for 128-wide grouped heads (K = V = the whole row,
example_sparse_flash_attn_gqa.py:13-295).

Semantics follow examples/sparse_flash_attention/example_sparse_flash_attn.py:18-292
(sm_scale default 1/sqrt(576), causal) and the paged variant
example_sparse_flash_attn_mask_pa.py:13-333 (``actual_seq_lengths``, block table,
``-1`` slots); the LSE convention is the V4 golden's
(examples/deepseek_v4/sparse_flash_mla/sparse_flash_mla_golden.py:149).  The
builder ``sparse_attention_fwd(heads, dim, tail_dim, topk, ...)`` keeps the
reference's builder signature (example_sparse_flash_attn.py:19-29) and returns a
callable that yields ``out`` only, as the reference kernel does.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import _lib

D_QK = 576
D_V = 512
D_GQA = 128

_KINDS = {torch.bfloat16: _lib.KIND_BF16, torch.float16: _lib.KIND_FP16}


def _lens(x: Optional[torch.Tensor], B: int, dev) -> Optional[torch.Tensor]:
    if x is None:
        return None
    t = torch.as_tensor(x).to(device=dev, dtype=torch.int32).reshape(-1).contiguous()
    if t.numel() != B:
        raise ValueError(f"actual sequence lengths must have B={B} entries, got {t.numel()}")
    return t


def sparse_mla_fwd(q: torch.Tensor, kv: torch.Tensor, indices: torch.Tensor, sm_scale: Optional[float] = None, *,
                   block_table: Optional[torch.Tensor] = None,
                   actual_seq_lengths_query: Optional[torch.Tensor] = None,
                   actual_seq_lengths_kv: Optional[torch.Tensor] = None,
                   is_causal: bool = True) -> Tuple[torch.Tensor, torch.Tensor]:
    """Sparse MLA forward; returns ``(out [B, S, H, 512], lse [B, S, H] fp32)``."""
    if q.dtype not in _KINDS:
        raise ValueError(f"q must be bfloat16 or float16, got {q.dtype}")
    if kv.dtype != q.dtype:
        raise ValueError(f"kv dtype {kv.dtype} must equal q dtype {q.dtype}")
    if indices.dtype != torch.int32:
        raise ValueError(f"indices must be int32, got {indices.dtype}")
    dev = _lib.require_device(q, kv, indices, block_table)
    if q.dim() != 4 or q.shape[-1] != D_QK:
        raise ValueError(f"q must be [B, S, H, {D_QK}], got {tuple(q.shape)}")
    B, S, H, _ = q.shape
    if kv.dim() != 4 or kv.shape[3] != D_QK:
        raise ValueError(f"kv must be [*, *, kv_group, {D_QK}], got {tuple(kv.shape)}")
    G = kv.shape[2]
    if G < 1 or H % G != 0 or (H // G) % 16 != 0 or H // G > 1024:
        raise ValueError(f"heads per KV group must be a multiple of 16 (<= 1024), got H={H}, kv_group={G}")
    if indices.dim() == 4:
        if indices.shape[2] != G:
            raise ValueError(f"indices have {indices.shape[2]} KV groups, kv has {G}")
        idx = indices if G > 1 else indices.reshape(B, S, indices.shape[3])
    elif indices.dim() == 3 and G == 1:
        idx = indices
    else:
        raise ValueError(f"indices must be [B, S, kv_group, topk] (or [B, S, topk]), got {tuple(indices.shape)}")
    if tuple(idx.shape[:2]) != (B, S):
        raise ValueError(f"indices batch/seq dims {tuple(idx.shape[:2])} do not match q {(B, S)}")
    topk = idx.shape[-1]
    for name, t in (("q", q), ("kv", kv), ("indices", idx)):
        _lib.require_contiguous(name, t)
    if block_table is not None:
        bt = block_table.to(torch.int32).contiguous()
        if bt.dim() != 2 or bt.shape[0] != B:
            raise ValueError(f"block_table must be [B, max_blocks], got {tuple(bt.shape)}")
        block_size, max_blocks = kv.shape[1], bt.shape[1]
        skv = max_blocks * block_size
    else:
        bt = None
        if kv.shape[0] != B:
            raise ValueError(f"kv batch {kv.shape[0]} does not match q batch {B}")
        block_size, max_blocks = 0, 0
        skv = kv.shape[1]
    if sm_scale is None:
        sm_scale = D_QK ** -0.5
    # Lengths stay on the device (no host sync); the kernel clamps them to
    # [0, S] and [0, Skv] before any address arithmetic.
    ql = _lens(actual_seq_lengths_query, B, dev)
    kl = _lens(actual_seq_lengths_kv, B, dev)
    out = torch.empty((B, S, H, D_V), dtype=q.dtype, device=dev)
    lse = torch.empty((B, S, H), dtype=torch.float32, device=dev)
    lib = _lib.load_library()
    if G > 1:
        ws_bytes = lib.dsa_sparse_attention_workspace_size(B, S, H, G, D_QK, topk)
        ws = torch.empty((max(ws_bytes, 1),), dtype=torch.uint8, device=dev)
        rc = lib.dsa_sparse_attention_fwd(_KINDS[q.dtype], _lib.ptr(q), _lib.ptr(kv), _lib.ptr(idx), _lib.ptr(bt),
                                          _lib.ptr(ql), _lib.ptr(kl), B, S, H, G, D_QK, D_V, skv, block_size,
                                          max_blocks, topk, float(sm_scale), 1 if is_causal else 0, _lib.ptr(out),
                                          _lib.ptr(lse), _lib.ptr(ws), ws_bytes, _lib.stream_handle(dev))
        _lib.check(rc, "dsa_sparse_attention_fwd")
        return out, lse
    ws_bytes = lib.dsa_sparse_mla_workspace_size(B, S, H, topk)
    ws = torch.empty((max(ws_bytes, 1),), dtype=torch.uint8, device=dev)
    rc = lib.dsa_sparse_mla_fwd(_KINDS[q.dtype], _lib.ptr(q), _lib.ptr(kv), _lib.ptr(idx), _lib.ptr(bt),
                                _lib.ptr(ql), _lib.ptr(kl), B, S, H, D_QK, D_V, skv, block_size, max_blocks, topk,
                                float(sm_scale), 1 if is_causal else 0, _lib.ptr(out), _lib.ptr(lse), _lib.ptr(ws),
                                ws_bytes, _lib.stream_handle(dev))
    _lib.check(rc, "dsa_sparse_mla_fwd")
    return out, lse


def sparse_gqa_fwd(q: torch.Tensor, kv: torch.Tensor, indices: torch.Tensor, sm_scale: Optional[float] = None, *,
                   actual_seq_lengths_query: Optional[torch.Tensor] = None,
                   actual_seq_lengths_kv: Optional[torch.Tensor] = None,
                   is_causal: bool = True) -> Tuple[torch.Tensor, torch.Tensor]:
    """Grouped 128-wide sparse attention (example_sparse_flash_attn_gqa.py:13-295);
    returns ``(out [B, S, H, 128], lse [B, S, H] fp32)``.

    q [B, S, H, 128], kv [B, Skv, G, 128] (K = V = the whole row), indices
    [B, S, G, topk] int32 (-1 = empty, topk <= 8192); query heads g*H/G ..
    (g+1)*H/G - 1 read KV head g.  sm_scale defaults to 128^-0.5; slot validity,
    causality and lengths as ``sparse_mla_fwd``.
    """
    if q.dtype not in _KINDS:
        raise ValueError(f"q must be bfloat16 or float16, got {q.dtype}")
    if kv.dtype != q.dtype:
        raise ValueError(f"kv dtype {kv.dtype} must equal q dtype {q.dtype}")
    if indices.dtype != torch.int32:
        raise ValueError(f"indices must be int32, got {indices.dtype}")
    dev = _lib.require_device(q, kv, indices)
    if q.dim() != 4 or q.shape[-1] != D_GQA:
        raise ValueError(f"q must be [B, S, H, {D_GQA}], got {tuple(q.shape)}")
    B, S, H, _ = q.shape
    if kv.dim() != 4 or kv.shape[0] != B or kv.shape[3] != D_GQA:
        raise ValueError(f"kv must be [{B}, Skv, kv_group, {D_GQA}], got {tuple(kv.shape)}")
    G = kv.shape[2]
    if G < 1 or H % G != 0 or H // G > 1024:
        raise ValueError(f"H={H} must be a multiple of kv_group={G} with at most 1024 heads per group")
    if indices.dim() != 4 or tuple(indices.shape[:3]) != (B, S, G):
        raise ValueError(f"indices must be [{B}, {S}, {G}, topk], got {tuple(indices.shape)}")
    topk = indices.shape[3]
    for name, t in (("q", q), ("kv", kv), ("indices", indices)):
        _lib.require_contiguous(name, t)
    if sm_scale is None:
        sm_scale = D_GQA ** -0.5  # example_sparse_flash_attn_gqa.py:30
    ql = _lens(actual_seq_lengths_query, B, dev)
    kl = _lens(actual_seq_lengths_kv, B, dev)
    out = torch.empty((B, S, H, D_GQA), dtype=q.dtype, device=dev)
    lse = torch.empty((B, S, H), dtype=torch.float32, device=dev)
    lib = _lib.load_library()
    rc = lib.dsa_sparse_attention_fwd(_KINDS[q.dtype], _lib.ptr(q), _lib.ptr(kv), _lib.ptr(indices), None,
                                      _lib.ptr(ql), _lib.ptr(kl), B, S, H, G, D_GQA, D_GQA, kv.shape[1], 0, 0, topk,
                                      float(sm_scale), 1 if is_causal else 0, _lib.ptr(out), _lib.ptr(lse), None, 0,
                                      _lib.stream_handle(dev))
    _lib.check(rc, "dsa_sparse_attention_fwd")
    return out, lse


def sparse_attention_fwd(heads: int, dim: int, tail_dim: int, topk: int, kv_stride: int = 1, kv_group: int = 1,
                         sm_scale: Optional[float] = None, is_causal: bool = True, block_I: int = 64, **_tuning):
    """Builder with the signature of example_sparse_flash_attn.py:19-29; returns ``kernel(q, kv, indices) -> out``.

    (dim, tail_dim) = (512, 64): the latent MLA kernel, kv [B, Skv, kv_group, 576];
    the paged form ``kernel(q, kv, indices, actual_q_len, actual_kv_len, block_table)``
    (example_sparse_flash_attn_mask_pa.py:440) is accepted too; paged indices may
    omit the batch dimension ([S, kv_group, topk]) as in that example (batch 1).
    (dim, tail_dim) = (128, 0): the grouped kernel of example_sparse_flash_attn_gqa.py:13-238,
    kv [B, Skv, kv_group, 128].
    """
    if (dim, tail_dim) not in ((D_V, D_QK - D_V), (D_GQA, 0)):
        raise ValueError(f"(dim, tail_dim) must be ({D_V}, {D_QK - D_V}) or ({D_GQA}, 0), got ({dim}, {tail_dim})")
    if kv_stride != 1:
        raise ValueError("kv_stride must be 1")
    if kv_group < 1 or heads % kv_group != 0:
        raise ValueError(f"heads {heads} must be a multiple of kv_group {kv_group}")
    head_kv = heads // kv_group
    if dim == D_V and head_kv % 16 != 0:
        raise ValueError(f"heads per KV group must be a multiple of 16, got {head_kv}")
    if head_kv > 64 and head_kv % 64 != 0:
        raise ValueError("head_kv should be a multiple of 64")  # example_sparse_flash_attn.py:65-66
    if not is_causal:
        raise ValueError("non-causal is not supported")  # example_sparse_flash_attn.py:32
    if topk % block_I != 0:
        raise ValueError("topk must be a multiple of block_I")  # example_sparse_flash_attn.py:33

    def kernel(q, kv, indices, actual_q_len=None, actual_kv_len=None, block_table=None):
        if q.shape[2] != heads:
            raise ValueError(f"q has {q.shape[2]} heads, builder expects {heads}")
        if kv.shape[2] != kv_group:
            raise ValueError(f"kv has {kv.shape[2]} KV groups, builder expects {kv_group}")
        idx = indices
        if block_table is not None and idx.dim() == 3:
            idx = idx.unsqueeze(0)
        if idx.shape[-1] != topk:
            raise ValueError(f"indices last dim {idx.shape[-1]} != topk {topk}")
        if dim == D_GQA:
            if block_table is not None:
                raise ValueError("the 128-wide grouped kernel takes a contiguous kv")
            out, _ = sparse_gqa_fwd(q, kv, idx, sm_scale, actual_seq_lengths_query=actual_q_len,
                                    actual_seq_lengths_kv=actual_kv_len, is_causal=True)
            return out
        out, _ = sparse_mla_fwd(q, kv, idx, sm_scale, block_table=block_table,
                                actual_seq_lengths_query=actual_q_len, actual_seq_lengths_kv=actual_kv_len,
                                is_causal=True)
        return out

    return kernel


def sparse_attn_tilelang(query, key, value, sparse_indices, scale_value, sparse_block_size,
                         actual_seq_lengths_query, actual_seq_lengths_kv, query_rope=None, key_rope=None,
                         layout_query="BSND", layout_kv="BSND", sparse_mode=3, block_table=None,
                         attention_mode=None):
    """The reference's torch_npu-style decode entry
    (examples/sparse_flash_attention/bench_sfa/sparse_flash_attn_pa_no_cv_pipeline.py:384-419):
    query [T, N, 512] with query_rope [T, N, 64]; key [blocks, block_size, 1, 512] with key_rope
    [blocks, block_size, 1, 64] (value is the key, as there); sparse_indices [T, 1, topk]; a paged
    cache through block_table.  Like the reference it joins each query / key with its rope part and
    runs the 576-wide kernel (causal when sparse_mode is 3); returns out [T, N, 512]."""
    del value, sparse_block_size, layout_query, layout_kv, attention_mode
    if query_rope is None or key_rope is None:
        raise ValueError("query_rope and key_rope are required (D = 512 + 64)")
    q = torch.cat((query.unsqueeze(0), query_rope.unsqueeze(0)), dim=-1).contiguous()
    kv = torch.cat((key, key_rope), dim=-1).contiguous()
    T = q.shape[1]
    idx = sparse_indices.to(torch.int32).reshape(1, T, 1, -1).contiguous()
    out, _ = sparse_mla_fwd(q, kv, idx, float(scale_value), block_table=block_table,
                            actual_seq_lengths_query=actual_seq_lengths_query,
                            actual_seq_lengths_kv=actual_seq_lengths_kv, is_causal=sparse_mode == 3)
    return out.squeeze(0)

