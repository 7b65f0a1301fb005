"""float64 torch restatement of the paged-attention closed form, on any device.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py). The same closed form as
``oracle.attention`` (follows _kernels_paged.py:317-357, _kernels_paged_verify.py:226-242,
_paged_adapter.py:658,753-754): for query row i of sequence b and q head h,

    O[b, i, h] = softmax_j( s * k_scale * q . K[slot(b, j), h // G] ) . V[slot(b, j), h // G] * v_scale

over the visible keys ``j < seq_b``, ``j <= P_b + i`` when causal, ``j >= P_b + i - window``
when ``window >= 0``. Written with torch so that full-size workloads (millions of keys)
are checked on the device that already holds them; every product and the softmax run in
float64. Pinned to ``oracle.attention`` (float64 numpy, itself pinned by SDPA, scalar
brute force and invariants) on seeded shapes in ``tests/test_oracle_attention.py``.
"""

from __future__ import annotations

from typing import Sequence

import torch


def attend(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor, seq_slots: Sequence[torch.Tensor],
           query_start_loc: Sequence[int], prefix_lens: Sequence[int], seq_lens: Sequence[int], *,
           softmax_scale: float, k_scale: float = 1.0, v_scale: float = 1.0, causal: bool = True,
           sliding_window: int = -1, sequences: Sequence[int] | None = None) -> torch.Tensor:
    """``q`` [T, Hq, D]; pools [slots, Hkv, D] in any dtype (fp8 pools are read with torch's
    cast, the reference's lookup table); ``seq_slots[b]`` the slot of every key position of
    sequence ``b``. Returns float64 [T, Hq, D] on q's device (rows of sequences not in
    ``sequences`` stay zero)."""
    T, Hq, D = q.shape
    Hkv = k_pool.shape[1]
    G = Hq // Hkv
    scale = float(softmax_scale) * float(k_scale)
    out = torch.zeros(T, Hq, v_pool.shape[-1], dtype=torch.float64, device=q.device)
    for b in (range(len(seq_lens)) if sequences is None else sequences):
        t0, t1 = int(query_start_loc[b]), int(query_start_loc[b + 1])
        n = int(seq_lens[b])
        if t1 <= t0 or n <= 0:
            continue
        idx = seq_slots[b][:n].to(device=k_pool.device, dtype=torch.long)
        kb = k_pool[idx].to(torch.float64)  # [n, Hkv, D]
        vb = v_pool[idx].to(torch.float64) * float(v_scale)
        E = t1 - t0
        P = int(prefix_lens[b])
        qpos = P + torch.arange(E, device=q.device)
        kpos = torch.arange(n, device=q.device)
        vis = torch.ones(E, n, dtype=torch.bool, device=q.device)
        if causal:
            vis &= kpos[None, :] <= qpos[:, None]
        if sliding_window >= 0:
            vis &= kpos[None, :] >= (qpos[:, None] - sliding_window)
        qb = q[t0:t1].to(torch.float64)  # [E, Hq, D]
        for h in range(Hkv):
            qh = qb[:, h * G:(h + 1) * G, :].reshape(E * G, D)
            kt = kb[:, h, :].t().contiguous()  # [D, n]
            s = (qh @ kt) * scale              # [E*G, n]; row r = (token r // G, head r % G)
            s = s.view(E, G, n).masked_fill(~vis[:, None, :], float("-inf"))
            m = s.amax(dim=-1, keepdim=True)
            m = torch.where(torch.isfinite(m), m, torch.zeros_like(m))
            p = torch.exp(s - m)
            den = p.sum(dim=-1, keepdim=True)
            o = (p.view(E * G, n) @ vb[:, h, :]).view(E, G, -1)
            out[t0:t1, h * G:(h + 1) * G, :] = torch.where(den > 0, o / den.clamp_min(1e-300), torch.zeros_like(o))
    return out


def rows_of_table(req_to_token: torch.Tensor, req_pool_indices, seq_lens) -> list:
    """``seq_slots`` of SGLang's layout: ``req_to_token[req_pool_indices[b], :seq_lens[b]]``."""
    rpi = [int(x) for x in req_pool_indices]
    return [req_to_token[rpi[b], :int(seq_lens[b])] for b in range(len(rpi))]
