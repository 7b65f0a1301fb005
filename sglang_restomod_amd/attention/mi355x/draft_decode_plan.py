"""Planning helpers for draft decode (sglang_restomod/attention/v100/draft_decode_plan.py:42-104).

``page_table_from_indices`` turns a flat ``kv_indptr`` / ``kv_indices`` list into the page
table plus per-row visible length of a page-granular decoder, entirely on device (no host
synchronisation, so it is safe inside a captured graph); the split-KV decoder here reads
such a list in place (``draft_decode.DraftRows.from_flat_lists``), and this conversion
serves callers that hold page tables. ``layer_shape_reason`` says why the decoder cannot
serve a layer, or None.
"""

from __future__ import annotations

import torch

PAGE_SIZE = 16        # head dims are multiples of this (draft_decode_plan.py:22, :93-94)
MAX_HEAD_DIM = 512    # the widest head dim the kernels take (ops.MAX_HEAD_DIM)


def page_table_from_indices(
    kv_indptr: torch.Tensor,
    kv_indices: torch.Tensor,
    page_table: torch.Tensor,
    seq_lens: torch.Tensor,
    page_size: int = 1,
) -> int:
    """Fill ``page_table[:rows]`` and ``seq_lens[:rows]``; return rows written (0 if the buffers are short).

    Row ``r`` owns ``kv_indices[indptr[r]:indptr[r+1]]``; its logical page ``p``
    is the page holding its token ``p * page_size``. Pages past the row's
    length are written as 0. An empty index list zeroes every row.
    """
    rows = int(kv_indptr.numel()) - 1
    if rows <= 0 or page_table.shape[0] < rows or seq_lens.shape[0] < rows:
        return 0
    if kv_indices.numel() == 0:
        page_table[:rows].zero_()
        seq_lens[:rows].zero_()
        return rows
    starts = kv_indptr[:rows].to(torch.int64)
    lengths = kv_indptr[1:rows + 1].to(torch.int64) - starts
    seq_lens[:rows].copy_(lengths.to(seq_lens.dtype))
    width = page_table.shape[1]
    first_token = torch.arange(width, dtype=torch.int64, device=kv_indices.device) * page_size
    flat = (starts[:, None] + first_token[None, :]).clamp_(max=kv_indices.numel() - 1)
    pages = torch.div(kv_indices[flat], page_size, rounding_mode="floor").to(torch.int32)
    inside = first_token[None, :] < lengths[:, None]
    page_table[:rows].copy_(torch.where(inside, pages, torch.zeros_like(pages)))
    return rows


def layer_shape_reason(layer) -> str | None:
    """Why the split-KV decoder cannot serve ``layer`` (None when it can)."""
    hq = int(getattr(layer, "tp_q_head_num", 0))
    hkv = int(getattr(layer, "tp_k_head_num", 0))
    qk = int(getattr(layer, "qk_head_dim", getattr(layer, "head_dim", 0)))
    vd = int(getattr(layer, "v_head_dim", qk))
    if hq <= 0 or hkv <= 0:
        return "no_head_count"
    if hq % hkv:
        return f"gqa_ratio(h={hq},hkv={hkv})"
    if qk != vd:
        return f"qk_dim({qk})!=v_dim({vd})"
    if qk % PAGE_SIZE:
        return f"dim({qk})_not_a_multiple_of_{PAGE_SIZE}"
    if qk <= 0 or qk > MAX_HEAD_DIM:
        return f"head_dim({qk})_not_in_1..{MAX_HEAD_DIM}"
    if getattr(layer, "is_cross_attention", False):
        return "cross_attention"
    if getattr(layer, "logit_cap", None) not in (None, 0, 0.0):
        return f"logit_cap({layer.logit_cap})"
    if getattr(layer, "xai_temperature_len", 0) > 0:
        return "xai_temperature"
    return None
