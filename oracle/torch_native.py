"""The torch-native SDPA form of the three attention modes, on the CPU.

This is the "reference's torch-native SDPA attention path" in the form the
reference's own GPU tests write it: gather each sequence's keys through the slot
table, upcast, repeat the kv heads for GQA and call
``torch.nn.functional.scaled_dot_product_attention`` with an explicit
causal-with-prefix mask (tests/test_attention_v100_gpu.py:28-46,
tests/test_native_draft_decode_gpu.py:42-60, tests/test_qsa_kernels_gpu.py:53-61).
fp8 KV is dequantized as ``raw.float() * scale`` (the per-tensor scale folded
into K and V is the same as scaling scores by ``k_scale`` and outputs by
``v_scale``, _paged_adapter.py:658,753-754).

It is the CPU baseline that ``bench.py`` times, and a second, independent
restatement that ``tests/test_oracle_attention.py`` cross-checks against the
float64 numpy oracle.
"""

from __future__ import annotations

import math
from typing import Optional, Sequence

import torch
import torch.nn.functional as F


def _dequant(pool: torch.Tensor, scale: float) -> torch.Tensor:
    out = pool.float()
    return out * scale if scale != 1.0 else out


def _sdpa(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float,
          mask: Optional[torch.Tensor]) -> torch.Tensor:
    """q [E, Hq, D], k/v [n, Hkv, D] -> [E, Hq, D]."""
    hq, hkv = q.shape[1], k.shape[1]
    rep = hq // hkv
    qq = q.transpose(0, 1).unsqueeze(0)
    kk = k.transpose(0, 1).unsqueeze(0).repeat_interleave(rep, dim=1)
    vv = v.transpose(0, 1).unsqueeze(0).repeat_interleave(rep, dim=1)
    out = F.scaled_dot_product_attention(qq, kk, vv, attn_mask=mask, scale=scale)
    return out.squeeze(0).transpose(0, 1)


def paged_attention(q, k_pool, v_pool, seq_slots: Sequence[torch.Tensor], query_start_loc,
                    prefix_lens, seq_lens, *, softmax_scale: float, k_scale: float = 1.0,
                    v_scale: float = 1.0, causal: bool = True, sliding_window: int = -1,
                    out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Per-sequence gather + fp32 SDPA. ``q`` [T, Hq, D]; pools [slots, Hkv, D]."""
    T, Hq, D = q.shape
    if out is None:
        out = torch.zeros(T, Hq, v_pool.shape[-1], dtype=torch.float32)
    for b in range(len(seq_lens)):
        t0, t1 = int(query_start_loc[b]), int(query_start_loc[b + 1])
        if t1 <= t0:
            continue
        n = int(seq_lens[b])
        if n == 0:
            out[t0:t1] = 0
            continue
        idx = seq_slots[b][:n].long()
        kb = k_pool[idx].float() * k_scale
        vb = v_pool[idx].float() * v_scale
        qb = q[t0:t1].float()
        P = int(prefix_lens[b])
        mask = None
        if causal or sliding_window >= 0:
            qpos = torch.arange(P, P + (t1 - t0))[:, None]
            kpos = torch.arange(n)[None, :]
            mask = torch.ones(t1 - t0, n, dtype=torch.bool)
            if causal:
                mask &= kpos <= qpos
            if sliding_window >= 0:
                mask &= kpos >= qpos - sliding_window
            mask = mask[None, None]
        out[t0:t1] = _sdpa(qb, kb, vb, softmax_scale, mask)
    return out


def decode(q, k_pool, v_pool, req_to_token, req_pool_indices, seq_lens, *, softmax_scale,
           k_scale=1.0, v_scale=1.0, sliding_window=-1, batch_subset=None):
    """``q`` [B, Hq, D]; no mask beyond the sequence length (decode sees its whole context)."""
    B = q.shape[0]
    rows = range(B) if batch_subset is None else batch_subset
    out = torch.zeros(B, q.shape[1], v_pool.shape[-1], dtype=torch.float32)
    for b in rows:
        n = int(seq_lens[b])
        if n == 0:
            continue
        idx = req_to_token[int(req_pool_indices[b]), :n].long()
        kb = k_pool[idx].float() * k_scale
        vb = v_pool[idx].float() * v_scale
        mask = None
        if sliding_window >= 0:
            kpos = torch.arange(n)
            mask = (kpos >= n - 1 - sliding_window)[None, None, None, :]
        out[b:b + 1] = _sdpa(q[b:b + 1].float(), kb, vb, softmax_scale, mask)
    return out


def extend(q, k_pool, v_pool, req_to_token, req_pool_indices, prefix_lens, extend_lens, *,
           softmax_scale, k_scale=1.0, v_scale=1.0, causal=True, sliding_window=-1):
    B = len(extend_lens)
    qsl = [0]
    for e in extend_lens:
        qsl.append(qsl[-1] + int(e))
    seq = [int(p) + int(e) for p, e in zip(prefix_lens, extend_lens)]
    slots = [req_to_token[int(req_pool_indices[b]), :seq[b]] for b in range(B)]
    return paged_attention(q, k_pool, v_pool, slots, qsl, prefix_lens, seq,
                           softmax_scale=softmax_scale, k_scale=k_scale, v_scale=v_scale,
                           causal=causal, sliding_window=sliding_window)


def default_scale(head_dim: int) -> float:
    return 1.0 / math.sqrt(head_dim)
