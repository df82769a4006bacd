"""CPU oracle for the DeepSeek Sparse Attention (DSA) inference path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product path imports this module:
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` use it, and only as the checker (or the timed CPU baseline).

It restates, in plain torch/numpy on the CPU, the reference's own goldens for
the three kernels of the path (all paths relative to the reference checkout):

* lightning indexer  -- ``examples/lightning_indexer/example_lightning_indexer.py:137-144``
  (``index_golden``) and ``examples/deepseek_v4/lightning_indexer.py:199-335``
  (``cpu_lightning_indexer``).  Superset: an optional per-key fp32 scale
  multiplies the head-weighted ReLU sum (fp8-e4m3 keys carry one scale per
  token); with ``k_scale=None`` it is exactly the reference formula.
* top-k selector     -- ``examples/topk_selector/example_topk_selector.py:57-58``
  with the tie rule of ``examples/deepseek_v4/lightning_indexer.py:317-325``
  (stable descending sort, lower index wins, selected scores <= -1e30 -> -1).
* sparse MLA forward -- gather form of
  ``examples/sparse_flash_attention/sfa_golden.py:64-199`` and
  ``examples/deepseek_v4/sparse_attention.py:171-198`` (``-1`` padding), with the
  natural-log LSE of
  ``examples/deepseek_v4/sparse_flash_mla/sparse_flash_mla_golden.py:149``;
  the dense scatter-mask form of
  ``examples/sparse_flash_attention/example_sparse_flash_attn.py:255-292`` is
  restated too, as an independent cross-check on tiny shapes.

How each function is pinned (see ``tests/test_oracle.py``):

* ``topk_stable``: the reference's own known-answer tests (``arange`` sort and
  top-k KATs, ``testing/python/language/test_tilelang_ascend_language_elementwise.py:4030-4248``),
  ``torch.topk`` on tie-free rows, brute force on tiny integer rows full of
  ties, constant rows and masked rows.
* ``indexer_logits``: explicit-loop brute force on tiny shapes, one-hot
  weights (isolates one head's ReLU(q.k)), linearity in the weights,
  homogeneity in the key scale, causal row lengths, and a one-hot q/k probe
  that fails on transposed operands.
* ``sparse_mla_fwd``: the dense-mask restatement, a single valid index
  (out = V row, lse = scale.q.k), equal scores (mean of V), permutation
  invariance, ``-1`` padding equal to dropping the slot, LSE against
  ``torch.logsumexp``.
* ``sparse_attention_grouped`` (KV groups, ``examples/sparse_flash_attention/example_sparse_flash_attn_gqa.py``):
  the dense restatement of that example's golden (``sparse_gqa_dense_ref``, which
  maps heads to groups by the golden's view / repeat_interleave rather than by
  slicing), equality with ``sparse_mla_fwd`` at one group, a permutation of the
  groups permuting the outputs, and a single valid index per group (out = that
  group's V row).
* ``fp8_quantize_per_token``: absmax maps to 448, representable values round
  trip exactly.
* ``act_quant`` (``examples/deepseek_v4/act_quant.py:118-142``, int8, extended
  to fp8 e4m3fn): a hand-worked int8 row with half-way cases, the 1e-4 floor
  of an all-zero row, power-of-two scales with ``round_scale``, the error bound
  |x - y * scale| <= scale / 2 (int8), and fp8 values on the e4m3 grid (and
  midpoints between grid points rounding to the even neighbour).
* ``v4_slots`` / ``sparse_flash_mla`` (DeepSeek V4 window + compressed
  attention with sinks, ``examples/deepseek_v4/sparse_flash_mla/sparse_flash_mla_golden.py:15-160``):
  hand-worked slot lists (window clipping, hca threshold, the csa walk that
  stops at the first -1 and skips entries past the threshold), a single-key
  closed form, ``torch.softmax`` / ``torch.logsumexp`` over scores with the
  sink appended, and a vanishing sink reducing to plain softmax attention.
* ``sparse_attn_sink`` (gathered-index attention with sinks,
  ``examples/deepseek_v4/sparse_attention.py:171-198``): all slots on one key
  (closed form kv * K e^s / (K e^s + e^sink)), the sink identity
  out = out_plain * sigmoid(lse_plain - sink) against the separately pinned
  ``sparse_mla_fwd``, -1 slots equal to dropping them, a duplicated slot equal
  to doubling that key's weight, and ``torch.softmax`` over scores with the
  sink appended.
* ``tnd_to_padded`` / ``padded_to_tnd`` (packed TND layout,
  ``examples/deepseek_v4/lightning_indexer.py:48-190``): a hand-worked row map
  with an empty batch, round trips both ways, and the zero fill of padding.
"""
from __future__ import annotations

import math
from typing import Optional, Sequence, Tuple

import numpy as np
import torch

NEG_INF = float("-inf")
# examples/deepseek_v4/lightning_indexer.py:322 -- selected scores at or below
# this threshold are reported as index -1.
INVALID_SCORE = -1e30
FP8_MAX = 448.0


# ----------------------------------------------------------------------------
# fp8 e4m3 (OCP "fn": no inf, max 448) per-token quantiser.  Not in the
# reference (its act_quant is int8, deepseek_v4/act_quant.py:33-92); this is the
# producer of the fp8 indexer inputs (q per tensor, k per token with scale absmax/448).
# ----------------------------------------------------------------------------
def fp8_quantize_per_token(x: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """x[..., D] float -> (x_fp8 [..., D] float8_e4m3fn, scale [...] fp32), scale = absmax/448."""
    xf = x.to(torch.float32)
    amax = xf.abs().amax(dim=-1)
    scale = torch.where(amax > 0, amax / FP8_MAX, torch.ones_like(amax))
    q = (xf / scale.unsqueeze(-1)).clamp(-FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn)
    return q, scale.to(torch.float32)


def act_quant(x: torch.Tensor, round_scale: bool = False,
              dtype: torch.dtype = torch.int8) -> Tuple[torch.Tensor, torch.Tensor]:
    """Per-row quantiser (examples/deepseek_v4/act_quant.py:118-142): amax =
    max(|x|) per row clamped to >= 1e-4, scale = amax / QMAX (round_scale:
    2^ceil(log2(amax / QMAX))), y = clamp(x / scale, -QMAX, QMAX) rounded half
    to even (int8, QMAX 127) or to nearest-even e4m3fn (fp8, QMAX 448).
    Returns (y shaped like x, scales [M, 1] or [B, S, 1])."""
    qmax = 127.0 if dtype == torch.int8 else FP8_MAX
    shape = x.shape
    x2 = x.reshape(-1, shape[-1]).float()
    amax = torch.clamp(x2.abs().amax(dim=1, keepdim=True), min=1e-4)
    scales = amax / qmax
    if round_scale:
        scales = torch.pow(2.0, torch.ceil(torch.log2(scales)))
    clipped = torch.clamp(x2 / scales, -qmax, qmax)
    if dtype == torch.int8:
        y = torch.round(clipped).to(torch.float16).to(torch.int8)
    else:
        y = clipped.to(torch.float8_e4m3fn)
    return y.reshape(shape), scales.reshape(shape[:-1] + (1,))


# ----------------------------------------------------------------------------
# Lightning indexer logits
# ----------------------------------------------------------------------------
def causal_valid_len(aq: int, ak: int, s1: int, sparse_mode: int) -> int:
    """Number of valid key positions for query row s1.

    examples/deepseek_v4/lightning_indexer.py:308-314: with sparse_mode 3 row s1
    sees keys s < ak - aq + s1 + 1; a non-positive bound falls back to ak.
    """
    if sparse_mode == 3:
        cl = ak - aq + s1 + 1
        return cl if cl > 0 else ak
    return ak


def indexer_logits(
    q: torch.Tensor,
    k: torch.Tensor,
    weights: torch.Tensor,
    k_scale: Optional[torch.Tensor] = None,
    *,
    actual_q_len: Optional[Sequence[int]] = None,
    actual_k_len: Optional[Sequence[int]] = None,
    sparse_mode: int = 3,
    row_chunk: int = 256,
    compute_dtype: torch.dtype = torch.float64,
) -> torch.Tensor:
    """logits[b, t, s] = k_scale[b, s] * sum_h w[b, t, h] * ReLU(q[b, t, h, :] . k[b, s, :]).

    q [B, S1, H, D] (fp8/fp16/bf16/fp32), k [B, S2, D] (or [B, S2, 1, D]),
    weights [B, S1, H], k_scale [B, S2] or None.  Returns fp32 [B, S1, S2] with
    masked positions (causal / beyond actual lengths / padded rows) = -inf.
    Follows examples/deepseek_v4/lightning_indexer.py:291-316 (einsum, ReLU,
    weighted head sum, causal mask) and example_lightning_indexer.py:137-142.
    Rows are processed in chunks so the [rows, H, S2] intermediate stays small
    (the reference materialises it whole, 34 GB at the largest config).
    ``compute_dtype`` float32 follows the reference's own fp32 arithmetic (used
    for the timed CPU baseline); the default float64 is the checker's.
    """
    if k.dim() == 4:
        k = k[:, :, 0, :]
    B, S1, H, D = q.shape
    S2 = k.shape[1]
    aq_l = [S1] * B if actual_q_len is None else [int(x) for x in actual_q_len]
    ak_l = [S2] * B if actual_k_len is None else [int(x) for x in actual_k_len]
    out = torch.full((B, S1, S2), NEG_INF, dtype=torch.float32)
    qf = q.to(torch.float32)
    kf = k.to(torch.float32)
    wf = weights.to(torch.float32)
    sc = None if k_scale is None else k_scale.to(torch.float32)
    for b in range(B):
        aq, ak = aq_l[b], ak_l[b]
        if aq == 0 or ak == 0:
            continue
        kb = kf[b, :ak].to(compute_dtype)  # [ak, D]
        for r0 in range(0, aq, row_chunk):
            r1 = min(aq, r0 + row_chunk)
            qb = qf[b, r0:r1].to(compute_dtype)  # [r, H, D]
            wb = wf[b, r0:r1].to(compute_dtype)  # [r, H]
            qk = torch.relu(torch.einsum("rhd,sd->rhs", qb, kb))
            score = torch.einsum("rhs,rh->rs", qk, wb)
            if sc is not None:
                score = score * sc[b, :ak].to(compute_dtype)[None, :]
            score = score.to(torch.float32)
            for i in range(r1 - r0):
                nv = causal_valid_len(aq, ak, r0 + i, sparse_mode)
                score[i, nv:] = NEG_INF
            out[b, r0:r1, :ak] = score
    return out


# ----------------------------------------------------------------------------
# Top-k selector
# ----------------------------------------------------------------------------
def topk_stable(scores: torch.Tensor, k: int, valid_len: Optional[Sequence[int]] = None
                ) -> Tuple[torch.Tensor, torch.Tensor]:
    """Row-wise top-k of fp32 scores [R, N] -> (idx int32 [R, k], values fp32 [R, k]).

    examples/deepseek_v4/lightning_indexer.py:317-325: a stable descending sort
    (ties -> lower index first), the first min(k, n) taken, any selected score
    <= -1e30 reported as index -1; slots past n hold -1 / -inf.  NaN scores
    are treated as -inf (a documented choice of this build).  Columns at or
    beyond ``valid_len[r]`` are excluded (equivalent to -inf).
    """
    x = scores.detach().to(torch.float32).cpu().clone()
    R, N = x.shape
    x = torch.where(torch.isnan(x), torch.full_like(x, NEG_INF), x)
    if valid_len is not None:
        cols = torch.arange(N)[None, :]
        vl = torch.as_tensor([int(v) for v in valid_len]).view(-1, 1)
        x = torch.where(cols < vl, x, torch.full_like(x, NEG_INF))
    idx = torch.full((R, k), -1, dtype=torch.int32)
    val = torch.full((R, k), NEG_INF, dtype=torch.float32)
    if N == 0 or R == 0:
        return idx, val
    kk = min(k, N)
    order = torch.argsort(-x, dim=1, stable=True)[:, :kk]
    topv = x.gather(1, order)
    topi = order.to(torch.int32)
    topi = torch.where(topv <= INVALID_SCORE, torch.full_like(topi, -1), topi)
    topv = torch.where(topv <= INVALID_SCORE, torch.full_like(topv, NEG_INF), topv)
    idx[:, :kk] = topi
    val[:, :kk] = topv
    return idx, val


def lightning_indexer(
    q: torch.Tensor,
    k: torch.Tensor,
    weights: torch.Tensor,
    k_scale: Optional[torch.Tensor] = None,
    *,
    actual_q_len: Optional[Sequence[int]] = None,
    actual_k_len: Optional[Sequence[int]] = None,
    sparse_count: int = 2048,
    sparse_mode: int = 3,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(indices [B, S1, 1, K] int32, values [B, S1, 1, K] fp32, logits [B, S1, S2]).

    examples/deepseek_v4/lightning_indexer.py:199-335 for the BSND layout.
    """
    logits = indexer_logits(q, k, weights, k_scale, actual_q_len=actual_q_len,
                            actual_k_len=actual_k_len, sparse_mode=sparse_mode)
    B, S1, S2 = logits.shape
    idx, val = topk_stable(logits.view(B * S1, S2), sparse_count)
    return idx.view(B, S1, 1, sparse_count), val.view(B, S1, 1, sparse_count), logits


# ----------------------------------------------------------------------------
# Packed (TND) layout: prefix sums <-> padded BSND rows
# ----------------------------------------------------------------------------
def prefix_to_lengths(cu: Sequence[int]) -> list:
    """Inclusive prefix sums -> per-batch lengths
    (examples/deepseek_v4/lightning_indexer.py:68-71, :136-138)."""
    cu = [int(x) for x in cu]
    return [cu[0]] + [cu[i] - cu[i - 1] for i in range(1, len(cu))]


def tnd_to_padded(x: torch.Tensor, cu: Sequence[int], S: Optional[int] = None) -> Tuple[torch.Tensor, list]:
    """Packed rows [T, ...] -> padded [B, S, ...] (zero fill) and the lengths.

    Batch b owns packed rows cu[b-1] .. cu[b]-1 (cu[-1] = 0); padded row (b, s)
    is packed row cu[b-1] + s for s < len[b].  S defaults to the longest length
    (examples/deepseek_v4/lightning_indexer.py:48-94, :127-163).
    """
    lens = prefix_to_lengths(cu)
    S = max(lens) if S is None else S
    out = torch.zeros((len(lens), S) + tuple(x.shape[1:]), dtype=x.dtype)
    start = 0
    for b, n in enumerate(lens):
        out[b, :n] = x[start:start + n]
        start += n
    return out, lens


def padded_to_tnd(x: torch.Tensor, lens: Sequence[int]) -> torch.Tensor:
    """Padded [B, S, ...] -> packed [sum(lens), ...], dropping padding rows
    (examples/deepseek_v4/lightning_indexer.py:166-190)."""
    parts = [x[b, :int(n)] for b, n in enumerate(lens)]
    return torch.cat(parts) if parts else x.reshape((0,) + tuple(x.shape[2:]))


def lightning_indexer_tnd(
    q: torch.Tensor,
    k: torch.Tensor,
    weights: torch.Tensor,
    cu_q: Sequence[int],
    k_scale: Optional[torch.Tensor] = None,
    *,
    cu_k: Optional[Sequence[int]] = None,
    actual_k_len: Optional[Sequence[int]] = None,
    sparse_count: int = 2048,
    sparse_mode: int = 3,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """TND query rows: (indices [T, 1, K], values [T, 1, K], logits [T, S2]).

    q [T, H, D], weights [T, H], cu_q prefix sums.  Keys either packed
    (k [Tk, D] or [Tk, 1, D], k_scale [Tk], cu_k prefix sums) or padded per
    batch (k [B, S2, D], k_scale [B, S2], actual_k_len lengths) -- the paged
    layout reduces to the latter.  The wrapper's conversion, then the BSND
    golden, then the packed output (examples/deepseek_v4/lightning_indexer.py:1257-1368).
    """
    qp, q_lens = tnd_to_padded(q, cu_q)
    wp, _ = tnd_to_padded(weights, cu_q)
    if cu_k is not None:
        if k.dim() == 3:
            k = k[:, 0, :]
        kp, k_lens = tnd_to_padded(k, cu_k)
        sp = None if k_scale is None else tnd_to_padded(k_scale, cu_k)[0]
    else:
        kp, sp = (k[:, :, 0, :] if k.dim() == 4 else k), k_scale
        k_lens = [int(x) for x in actual_k_len]
    logits = indexer_logits(qp, kp, wp, sp, actual_q_len=q_lens, actual_k_len=k_lens, sparse_mode=sparse_mode)
    B, S1, S2 = logits.shape
    idx, val = topk_stable(logits.reshape(B * S1, S2), sparse_count)
    idx, val = idx.view(B, S1, sparse_count), val.view(B, S1, sparse_count)
    return (padded_to_tnd(idx, q_lens).unsqueeze(1), padded_to_tnd(val, q_lens).unsqueeze(1),
            padded_to_tnd(logits, q_lens))


# ----------------------------------------------------------------------------
# Sparse MLA forward
# ----------------------------------------------------------------------------
def _gather_rows(kv: torch.Tensor, b: int, idx: torch.Tensor,
                 block_table: Optional[torch.Tensor], block_size: int) -> torch.Tensor:
    """KV rows for batch b at logical positions idx (all >= 0)."""
    if block_table is None:
        return kv[b, idx.long(), 0, :]
    blk = block_table[b, (idx // block_size).long()].long()
    return kv[blk, (idx % block_size).long(), 0, :]


def sparse_mla_fwd(
    q: torch.Tensor,
    kv: torch.Tensor,
    indices: torch.Tensor,
    sm_scale: Optional[float] = None,
    *,
    d_v: int = 512,
    block_table: Optional[torch.Tensor] = None,
    actual_seq_lengths_query: Optional[Sequence[int]] = None,
    actual_seq_lengths_kv: Optional[Sequence[int]] = None,
    is_causal: bool = True,
    compute_dtype: torch.dtype = torch.float64,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Sparse MLA forward, gather form.  Returns (out fp32 [B,S,H,d_v], lse fp32 [B,S,H]).

    q [B, S, H, Dqk]; kv [B, Skv, 1, Dqk] or, with ``block_table`` [B, nblk],
    a paged pool [num_blocks, block_size, 1, Dqk]; indices [B, S, 1, topk]
    int32.  V is kv[..., :d_v] (example_sparse_flash_attn.py:270-271).

    Slot j of row (b, s) is valid iff idx >= 0, idx < kv_len[b] and, when
    causal, idx <= kv_len[b] - q_len[b] + s (example_sparse_flash_attn_mask_pa.py:221-224,
    sfa_golden.py:85-101).  Scores are scale * q.k in fp32
    (sfa_golden.py:183-184), softmax over the valid slots, out = P V
    (sfa_golden.py:193), lse = max + ln(sum exp) in natural log
    (sparse_flash_mla_golden.py:149).  A row with no valid slot gives out = 0,
    lse = -inf.  Duplicate indices in a row are a precondition violation.
    """
    B, S, H, Dqk = q.shape
    if sm_scale is None:
        sm_scale = Dqk ** -0.5  # example_sparse_flash_attn.py:36
    paged = block_table is not None
    if paged:
        block_size = kv.shape[1]
        skv_default = block_table.shape[1] * block_size
    else:
        block_size = 0
        skv_default = kv.shape[1]
    ql = [S] * B if actual_seq_lengths_query is None else [int(x) for x in actual_seq_lengths_query]
    kl = [skv_default] * B if actual_seq_lengths_kv is None else [int(x) for x in actual_seq_lengths_kv]
    idx_all = indices.reshape(B, S, -1).to(torch.int64).cpu()
    out = torch.zeros((B, S, H, d_v), dtype=torch.float32)
    lse = torch.full((B, S, H), NEG_INF, dtype=torch.float32)
    qf = q.to(torch.float32)
    kvf = kv.to(torch.float32)
    for b in range(B):
        for s in range(ql[b]):
            row = idx_all[b, s]
            valid = (row >= 0) & (row < kl[b])
            if is_causal:
                valid &= row <= kl[b] - ql[b] + s
            sel = row[valid]
            if sel.numel() == 0:
                continue
            assert torch.unique(sel).numel() == sel.numel(), "indices must be unique per row"
            kr = _gather_rows(kvf, b, sel, block_table if paged else None, block_size).to(compute_dtype)
            qr = qf[b, s].to(compute_dtype)  # [H, Dqk]
            sc = (qr @ kr.T) * sm_scale  # [H, n]
            m = sc.amax(dim=1, keepdim=True)
            p = torch.exp(sc - m)
            l = p.sum(dim=1, keepdim=True)
            out[b, s] = ((p / l) @ kr[:, :d_v]).to(torch.float32)
            lse[b, s] = (m + torch.log(l)).squeeze(1).to(torch.float32)
    return out, lse


def sparse_mla_dense_ref(q: torch.Tensor, kv: torch.Tensor, indices: torch.Tensor,
                         q_start_index_s: Optional[int] = None, sm_scale: Optional[float] = None,
                         d_v: int = 512) -> torch.Tensor:
    """Dense scatter-mask restatement of example_sparse_flash_attn.py:255-292 (kv_stride 1).

    Builds the [B, S, Skv] boolean mask from the indices (-1 slots dropped), ANDs
    the causal mask q_start + t >= j, and runs a dense masked softmax.  Used on
    tiny shapes only, as an independent check of ``sparse_mla_fwd``.
    """
    qf = q.to(torch.float64)
    kvf = kv.to(torch.float64)[:, :, 0, :]
    B, S, H, Dqk = q.shape
    Skv = kv.shape[1]
    if q_start_index_s is None:
        q_start_index_s = Skv - S
    if sm_scale is None:
        sm_scale = Dqk ** -0.5
    idx = indices.reshape(B, S, -1).long()
    safe = torch.where(idx < 0, torch.full_like(idx, Skv), idx)
    mask = torch.zeros(B, S, Skv + 1, dtype=torch.bool).scatter(2, safe, True)[..., :Skv]
    causal = torch.arange(q_start_index_s, q_start_index_s + S).view(-1, 1) >= torch.arange(Skv).view(1, -1)
    mask &= causal.view(1, S, Skv)
    score = torch.einsum("bshd,bnd->bshn", qf, kvf)
    score = score.masked_fill(~mask.view(B, S, 1, Skv), float("-inf")) * sm_scale
    p = score.softmax(dim=-1)
    p = torch.nan_to_num(p, nan=0.0)
    return torch.einsum("bshn,bnd->bshd", p, kvf[..., :d_v]).to(torch.float32)


def sparse_attention_grouped(
    q: torch.Tensor,
    kv: torch.Tensor,
    indices: torch.Tensor,
    sm_scale: Optional[float] = None,
    *,
    d_v: int,
    block_table: Optional[torch.Tensor] = None,
    actual_seq_lengths_query: Optional[Sequence[int]] = None,
    actual_seq_lengths_kv: Optional[Sequence[int]] = None,
    is_causal: bool = True,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Sparse attention over G KV heads: (out fp32 [B, S, H, d_v], lse fp32 [B, S, H]).

    kv [B, Skv, G, Dqk] (or, with ``block_table``, a pool [num_blocks, block_size, G, Dqk]);
    indices [B, S, G, topk].  Query heads g*Hg .. (g+1)*Hg - 1 (Hg = H / G) read KV head g
    through indices[:, :, g] (example_sparse_flash_attn.py:41-46 shapes; the goldens'
    q.view(b, sq, g, h, d), example_sparse_flash_attn_gqa.py:276-283).  Groups do not
    interact: each is ``sparse_mla_fwd`` on its own slices, with the default scale
    Dqk^-0.5 of the whole row (example_sparse_flash_attn_gqa.py:30).
    """
    B, S, H, Dqk = q.shape
    G = kv.shape[2]
    assert H % G == 0, "H must be a multiple of the KV groups"
    Hg = H // G
    if sm_scale is None:
        sm_scale = Dqk ** -0.5
    idx = indices.reshape(B, S, G, -1)
    out = torch.zeros((B, S, H, d_v), dtype=torch.float32)
    lse = torch.full((B, S, H), NEG_INF, dtype=torch.float32)
    for g in range(G):
        o, l = sparse_mla_fwd(q[:, :, g * Hg:(g + 1) * Hg], kv[:, :, g:g + 1], idx[:, :, g:g + 1], sm_scale,
                              d_v=d_v, block_table=block_table, actual_seq_lengths_query=actual_seq_lengths_query,
                              actual_seq_lengths_kv=actual_seq_lengths_kv, is_causal=is_causal)
        out[:, :, g * Hg:(g + 1) * Hg] = o
        lse[:, :, g * Hg:(g + 1) * Hg] = l
    return out, lse


def sparse_gqa_dense_ref(q: torch.Tensor, kv: torch.Tensor, indices: torch.Tensor,
                         q_start_index_s: Optional[int] = None, sm_scale: Optional[float] = None,
                         d_v: Optional[int] = None) -> torch.Tensor:
    """Dense scatter-mask restatement of the grouped golden
    ``ref_sparse_attention_fwd_interface_gqa`` (example_sparse_flash_attn_gqa.py:241-283,
    kv_stride 1): a [B, G, S, Skv] mask per KV head from its index rows (-1 slots dropped)
    AND the causal mask q_start + t >= j, scores of q viewed as [B, S, G, Hg, D], and the
    probabilities of query head h applied to KV head h // Hg (the golden's
    ``repeat_interleave``).  d_v defaults to the whole row (K = V).  Tiny shapes only:
    an independent check of ``sparse_attention_grouped``.
    """
    qf = q.to(torch.float64)
    kvf = kv.to(torch.float64)
    B, S, H, D = q.shape
    Skv, G = kv.shape[1], kv.shape[2]
    Hg = H // G
    d_v = D if d_v is None else d_v
    if q_start_index_s is None:
        q_start_index_s = Skv - S
    if sm_scale is None:
        sm_scale = D ** -0.5
    idx = indices.reshape(B, S, G, -1).long().transpose(1, 2)  # [B, G, S, topk]
    safe = torch.where(idx < 0, torch.full_like(idx, Skv), idx)
    mask = torch.zeros(B, G, S, Skv + 1, dtype=torch.bool).scatter(3, safe, True)[..., :Skv]
    causal = torch.arange(q_start_index_s, q_start_index_s + S).view(-1, 1) >= torch.arange(Skv).view(1, -1)
    mask &= causal.view(1, 1, S, Skv)
    score = torch.einsum("bqghd,bkgd->bghqk", qf.view(B, S, G, Hg, D), kvf)
    score = score.masked_fill(~mask.view(B, G, 1, S, Skv), float("-inf")) * sm_scale
    p = torch.nan_to_num(score.softmax(dim=-1), nan=0.0).reshape(B, H, S, Skv)
    v = kvf[..., :d_v].repeat_interleave(Hg, dim=2)  # [B, Skv, H, d_v]
    return torch.einsum("bhqs,bshd->bqhd", p, v).to(torch.float32)


# ----------------------------------------------------------------------------
# DeepSeek V4 sparse flash MLA (window over original KV + compressed KV, sinks)
# ----------------------------------------------------------------------------
def v4_slots(s_global: int, *, win_left: int, cmp_ratio: Optional[int] = None, dense_cmp: bool = False,
             sel: Optional[Sequence[int]] = None) -> Tuple[list, list]:
    """(original positions, compressed positions) one query row attends to.

    Window: max(s_global - win_left, 0) .. s_global (ori_win_right = 0,
    sparse_flash_mla_golden.py:103-105); none when s_global < 0.  Compressed,
    with threshold = floor((s_global + 1) / cmp_ratio) (cmp_mask_mode 3, :27-29):
    ``dense_cmp`` ("hca") takes 0 .. threshold - 1 (:121-123); ``sel`` ("csa")
    walks the first min(len(sel), threshold) entries, stops at the first -1 and
    skips entries >= threshold (:31-45, sparse_block_size 1).  Entries below -1
    are skipped (the golden would wrap them around as Python indices).
    """
    if s_global < 0:
        return [], []
    ori = list(range(max(s_global - win_left, 0), s_global + 1))
    cmp: list = []
    if cmp_ratio is not None and (dense_cmp or sel is not None):
        thr = (s_global + 1) // cmp_ratio
        if dense_cmp:
            cmp = list(range(thr))
        else:
            for i in range(min(len(sel), thr)):
                tid = int(sel[i])
                if tid == -1:
                    break
                if 0 <= tid < thr:
                    cmp.append(tid)
    return ori, cmp


def unpack_paged(pool: torch.Tensor, table: torch.Tensor, length: int, b: int) -> torch.Tensor:
    """Logical rows 0 .. length-1 of batch b from a paged pool [blocks, bs, 1, D]
    (sparse_flash_mla_golden.py:199-219)."""
    bs = pool.shape[1]
    pos = torch.arange(length)
    blk = table[b].to(torch.int64)[pos // bs]
    return pool[blk, pos % bs, 0]


def _golden_row(q, ori_k, cmp_k, sinks, scale, p_dtype, tile=512):
    """One row the golden's way (sparse_flash_mla_golden.py:125-150), float32."""
    H, D = q.shape
    row_max = sinks.clone() if sinks is not None else torch.full((H,), float("-inf"))
    row_sum = torch.ones(H) if sinks is not None else torch.zeros(H)
    acc = torch.zeros((H, D))
    for part in (ori_k, cmp_k):
        if part is None or part.shape[0] == 0:
            continue
        for t0 in range(0, part.shape[0], tile):
            k = part[t0:t0 + tile]
            score = (q @ k.T) * scale
            old = row_max
            row_max = torch.maximum(row_max, score.amax(dim=1))
            alpha = torch.exp(old - row_max)
            p = torch.exp(score - row_max[:, None])
            row_sum = alpha * row_sum + p.sum(dim=1)
            acc = acc * alpha[:, None] + p.to(p_dtype).float() @ k
    if not torch.isfinite(row_max).all():
        return torch.zeros((H, D), dtype=torch.float64), torch.full((H,), float("-inf"), dtype=torch.float64)
    return ((acc / row_sum[:, None]).to(p_dtype).double(), (row_max + torch.log(row_sum)).double())


def sparse_flash_mla(
    q: torch.Tensor,
    cu_seqlens_q: Sequence[int],
    seqused_kv: Sequence[int],
    ori_kv: torch.Tensor,
    ori_block_table: torch.Tensor,
    sinks: Optional[torch.Tensor],
    softmax_scale: float,
    *,
    cmp_kv: Optional[torch.Tensor] = None,
    cmp_block_table: Optional[torch.Tensor] = None,
    cmp_sparse_indices: Optional[torch.Tensor] = None,
    cmp_ratio: Optional[int] = None,
    ori_win_left: int = 127,
    golden_p_dtype: Optional[torch.dtype] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """V4 attention over packed query rows: (out fp32 [T, H, D], lse fp32 [T, H]).

    q [T, H, D]; cu_seqlens_q [B+1]; paged caches [blocks, bs, 1, D] with
    tables [B, n]; cmp_sparse_indices [T, 1, K] or [T, K].  For each row the
    slot list of ``v4_slots`` is gathered (K = V = the row), scores are
    scale * q.k, and the sink of head h enters the softmax as one more logit
    with no value row: out = sum_j p_j v_j, p = exp(s - m) / (sum exp(s - m)
    + exp(sink - m)), lse = m + ln(denominator)
    (sparse_flash_mla_golden.py:125-150, sinks_softmax_reference :163-185).
    Rows past cu_seqlens_q[-1] stay 0 (out and lse).

    Exact (float64) by default.  With ``golden_p_dtype`` it instead follows
    the golden's own arithmetic (:125-150): float32, online softmax over
    512-key tiles (original rows, then compressed), P rounded to that dtype
    before P V, out rounded to it at the end -- the reference's error profile,
    used to calibrate how close a bf16 kernel can be to the exact result.
    """
    T, H, D = q.shape
    out = torch.zeros((T, H, D), dtype=torch.float64)
    lse = torch.zeros((T, H), dtype=torch.float64)
    sk = None if sinks is None else sinks.to(torch.float64).view(H, 1)
    cu = [int(x) for x in cu_seqlens_q]
    sel_all = None
    if cmp_sparse_indices is not None:
        sel_all = cmp_sparse_indices.reshape(cmp_sparse_indices.shape[0], -1)
    for b in range(len(cu) - 1):
        aq, akv = cu[b + 1] - cu[b], int(seqused_kv[b])
        if aq <= 0:
            continue
        ori_rows = unpack_paged(ori_kv, ori_block_table, akv, b).to(torch.float64)
        cmp_rows = None
        if cmp_kv is not None and cmp_ratio is not None:
            cmp_rows = unpack_paged(cmp_kv, cmp_block_table, akv // cmp_ratio, b).to(torch.float64)
        for s in range(aq):
            t = cu[b] + s
            sg = akv - aq + s
            sel = None if sel_all is None else sel_all[t].tolist()
            o_pos, c_pos = v4_slots(sg, win_left=ori_win_left, cmp_ratio=cmp_ratio if cmp_rows is not None else None,
                                    dense_cmp=cmp_rows is not None and sel is None, sel=sel)
            keys = [ori_rows[o_pos]]
            if c_pos:
                keys.append(cmp_rows[c_pos])
            kmat = torch.cat(keys) if keys else torch.zeros((0, D), dtype=torch.float64)
            if golden_p_dtype is not None:
                out[t], lse[t] = _golden_row(q[t].float(), ori_rows[o_pos].float(),
                                             cmp_rows[c_pos].float() if c_pos else None,
                                             None if sinks is None else sinks.float(), softmax_scale, golden_p_dtype)
                continue
            qt = q[t].to(torch.float64)
            score = (qt @ kmat.T) * softmax_scale                       # [H, n]
            logits = score if sk is None else torch.cat([score, sk], dim=1)
            if logits.shape[1] == 0:
                out[t] = 0.0
                lse[t] = float("-inf")
                continue
            m = logits.amax(dim=1, keepdim=True)
            e = torch.exp(logits - m)
            denom = e.sum(dim=1, keepdim=True)
            p = e[:, :score.shape[1]] / denom
            out[t] = p @ kmat
            lse[t] = (m + torch.log(denom)).squeeze(1)
    return out.to(torch.float32), lse.to(torch.float32)


def sparse_attn_sink(
    q: torch.Tensor,
    kv: torch.Tensor,
    attn_sink: Optional[torch.Tensor],
    topk_idxs: torch.Tensor,
    softmax_scale: float,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """V4 gathered-index attention with sinks: (out fp32 [b, m, h, d], lse fp32 [b, m, h]).

    Restates ``examples/deepseek_v4/sparse_attention.py:171-198``: q [b, m, h, d],
    kv [b, n, d] (K = V), topk_idxs [b, m, topk].  Slot j of row (b, t) holds
    kv[b, idx] when idx != -1 (:171-177; duplicates count once per slot) and is
    masked to -inf otherwise (:195); scores are scale * q.k; the sink of head h is
    one more logit with no value row (:180-188): p = exp(s - M) / (sum exp(s - M)
    + exp(sink - M)) with M the max over the slots; out = p V (:198).  lse = natural
    log of the full denominator (sink included), in the convention of
    ``sparse_flash_mla_golden.py:149`` (the reference kernel writes no LSE).

    Out-of-contract rows, defined here the way the HIP kernel handles them: an
    index outside [0, n) is masked like -1 (the reference would read out of
    bounds), and a row with no valid slot gives out = 0, lse = sink (the
    reference's golden is NaN there: exp(-inf - -inf)).  Exact, in float64.
    """
    B, M, H, D = q.shape
    out = torch.zeros((B, M, H, D), dtype=torch.float64)
    lse = torch.zeros((B, M, H), dtype=torch.float64)
    n = kv.shape[1]
    sk = None if attn_sink is None else attn_sink.to(torch.float64).reshape(H, 1)
    idx_all = topk_idxs.to(torch.int64).cpu()
    kvd = kv.to(torch.float64)
    for b in range(B):
        for t in range(M):
            row = idx_all[b, t]
            sel = row[(row >= 0) & (row < n)]
            kmat = kvd[b, sel]                                          # [nv, d]
            score = (q[b, t].to(torch.float64) @ kmat.T) * softmax_scale  # [H, nv]
            logits = score if sk is None else torch.cat([score, sk], dim=1)
            if logits.shape[1] == 0:
                lse[b, t] = float("-inf")
                continue
            mx = logits.amax(dim=1, keepdim=True)
            e = torch.exp(logits - mx)
            denom = e.sum(dim=1, keepdim=True)
            out[b, t] = (e[:, :score.shape[1]] / denom) @ kmat
            lse[b, t] = (mx + torch.log(denom)).squeeze(1)
    return out.to(torch.float32), lse.to(torch.float32)


# ----------------------------------------------------------------------------
# Seeded input generators for the benchmark configurations
# ----------------------------------------------------------------------------
def _gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def causal_sparse_indices(B: int, S: int, Skv: int, topk: int, seed: int,
                          q_start: Optional[int] = None) -> torch.Tensor:
    """indices [B, S, 1, topk] int32: row t draws min(topk, q_start+t+1) distinct
    positions from [0, q_start+t] without replacement, -1 padded.

    Vectorised: top-k of i.i.d. uniform keys over the causal range is a uniform
    sample without replacement.
    """
    if q_start is None:
        q_start = Skv - S
    g = _gen(seed)
    out = torch.full((B, S, 1, topk), -1, dtype=torch.int32)
    chunk = max(1, (1 << 24) // max(Skv, 1))
    for b in range(B):
        for r0 in range(0, S, chunk):
            r1 = min(S, r0 + chunk)
            u = torch.rand((r1 - r0, Skv), generator=g)
            lim = torch.arange(r0, r1).view(-1, 1) + q_start + 1
            u = torch.where(torch.arange(Skv).view(1, -1) < lim, u, torch.full_like(u, -1.0))
            kk = min(topk, Skv)
            v, i = torch.topk(u, kk, dim=1)
            i = torch.where(v >= 0, i, torch.full_like(i, -1)).to(torch.int32)
            out[b, r0:r1, 0, :kk] = i
    return out
