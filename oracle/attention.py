"""Float64 restatement of the paged-attention semantics (decode, extend, verify).

Closed form (the one the reference's own GPU tests check their kernels with):
for query row ``t`` of sequence ``b`` (local index ``i = t - qsl[b]``) and query
head ``h``, with ``G = Hq // Hkv`` and visible key positions ``j``,

    O[t, h] = v_scale * softmax_j( s * q[t, h] . K[slot(b, j), h // G] ) @ V[slot(b, j), h // G]
    s       = softmax_scale * k_scale

* key visibility (sglang_restomod/attention/v100/tilelang/_kernels_paged.py:317-357):
  ``j < seq_lens[b]``; if causal also ``j <= prefix[b] + i``; if a window
  ``W >= 0`` is set also ``j >= prefix[b] + i - W`` (a left bound only, also
  for non-causal layers, masks.py:22-28).
* the head mapping ``h // G`` (_kernels_paged.py:265, _kernels_paged_decode.py:108,
  tests/test_native_draft_decode_gpu.py:42-60).
* ``slot(b, j)`` is ``req_to_token[req_pool_indices[b], j]`` for a token pool
  (page size 1), or ``table[b, j // ps] * ps + j % ps`` for a page table
  (_kernels_paged.py:309-315).
* scale convention: scores use ``softmax_scale * k_scale``
  (_paged_adapter.py:658), outputs are multiplied by ``v_scale`` (:753-754).
* decode is the ``i = 0``, ``prefix = seq_len - 1`` case; linear-chain verify
  is extend with ``E = draft_token_num`` and ``prefix = seq_lens``
  (flash_attn_v100_backend.py:594-598).
* a row that sees no key returns zeros: the grouped decoder writes LSE -2**30
  and a zero partial for an empty split and the combine keeps it at zero
  (_kernels_paged_decode.py:221-248, 287-310).

Pinned by ``tests/test_oracle_attention.py``: against
``torch.nn.functional.scaled_dot_product_attention`` (library routine) on
random inputs with explicit masks, against a scalar brute-force loop on tiny
shapes, and against invariants that a dropped term / wrong index / transposed
operand breaks: one visible key returns that V row, equal scores return the
mean of V, a permuted slot table gives the identity-layout answer, GQA maps
head h to kv head h // G (not h % Hkv), the causal bound is inclusive.
"""

from __future__ import annotations

from typing import Optional, Sequence

import numpy as np


def slots_from_token_table(req_to_token: np.ndarray, row: int, length: int) -> np.ndarray:
    """Token-pool slots of the first ``length`` positions of request row ``row``."""
    return np.asarray(req_to_token[row, :length], dtype=np.int64)


def slots_from_page_table(page_table: np.ndarray, b: int, length: int, page_size: int) -> np.ndarray:
    """Physical token rows through a page table: ``table[b, j // ps] * ps + j % ps``."""
    j = np.arange(length, dtype=np.int64)
    pages = np.asarray(page_table[b], dtype=np.int64)[j // page_size]
    return pages * page_size + (j % page_size)


def _attend(q_rows: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float,
            lo: np.ndarray, hi: np.ndarray) -> np.ndarray:
    """Rows of ``q_rows`` [R, D] over keys ``k``/``v`` [n, D]; row r sees [lo[r], hi[r])."""
    n = k.shape[0]
    out = np.zeros((q_rows.shape[0], v.shape[1]), dtype=np.float64)
    if n == 0:
        return out
    scores = (q_rows @ k.T) * scale  # [R, n]
    pos = np.arange(n)[None, :]
    visible = (pos >= lo[:, None]) & (pos < hi[:, None])
    any_visible = visible.any(axis=1)
    scores = np.where(visible, scores, -np.inf)
    m = np.max(np.where(any_visible[:, None], scores, 0.0), axis=1, keepdims=True)
    m = np.where(np.isfinite(m), m, 0.0)
    p = np.where(visible, np.exp(scores - m), 0.0)
    denom = p.sum(axis=1, keepdims=True)
    out = np.where(any_visible[:, None], (p @ v) / np.where(denom == 0, 1.0, denom), 0.0)
    return out


def paged_attention(
    q: np.ndarray,
    k_pool: np.ndarray,
    v_pool: np.ndarray,
    seq_slots: Sequence[np.ndarray],
    query_start_loc: Sequence[int],
    prefix_lens: Sequence[int],
    seq_lens: Sequence[int],
    *,
    softmax_scale: float,
    k_scale: float = 1.0,
    v_scale: float = 1.0,
    causal: bool = True,
    sliding_window: int = -1,
) -> np.ndarray:
    """General form: ``q`` [T, Hq, D]; pools [slots, Hkv, D] (already dequantized).

    ``seq_slots[b]`` holds the token-pool slot of every key position of
    sequence ``b`` (at least ``seq_lens[b]`` entries). Returns float64 [T, Hq, D].
    """
    q = np.asarray(q, dtype=np.float64)
    T, Hq, D = q.shape
    Hkv = k_pool.shape[1]
    if Hq % Hkv:
        raise ValueError("query heads must be a multiple of kv heads")
    G = Hq // Hkv
    scale = float(softmax_scale) * float(k_scale)
    out = np.zeros((T, Hq, v_pool.shape[2]), dtype=np.float64)
    for b in range(len(seq_lens)):
        t0, t1 = int(query_start_loc[b]), int(query_start_loc[b + 1])
        if t1 <= t0:
            continue
        n = int(seq_lens[b])
        slots = np.asarray(seq_slots[b][:n], dtype=np.int64)
        kb = np.asarray(k_pool[slots], dtype=np.float64)  # [n, Hkv, D]
        vb = np.asarray(v_pool[slots], dtype=np.float64)
        i = np.arange(t1 - t0)
        P = int(prefix_lens[b])
        hi = np.minimum(n, P + i + 1) if causal else np.full_like(i, n)
        lo = np.maximum(0, P + i - sliding_window) if sliding_window >= 0 else np.zeros_like(i)
        for h in range(Hkv):
            rows = q[t0:t1, h * G:(h + 1) * G, :].reshape(-1, D)  # [(E*G), D], row = i*G + g
            lo_r = np.repeat(lo, G)
            hi_r = np.repeat(hi, G)
            o = _attend(rows, kb[:, h, :], vb[:, h, :], scale, lo_r, hi_r)
            out[t0:t1, h * G:(h + 1) * G, :] = o.reshape(t1 - t0, G, -1)
    return out * float(v_scale)


def decode(
    q: np.ndarray,
    k_pool: np.ndarray,
    v_pool: np.ndarray,
    req_to_token: np.ndarray,
    req_pool_indices: Sequence[int],
    seq_lens: Sequence[int],
    *,
    softmax_scale: float,
    k_scale: float = 1.0,
    v_scale: float = 1.0,
    sliding_window: int = -1,
) -> np.ndarray:
    """One query token per sequence: ``q`` [B, Hq, D] -> [B, Hq, D]."""
    B = q.shape[0]
    slots = [slots_from_token_table(req_to_token, int(req_pool_indices[b]), int(seq_lens[b]))
             for b in range(B)]
    seq = [int(s) for s in seq_lens]
    return paged_attention(
        q, k_pool, v_pool, slots, list(range(B + 1)), [max(s - 1, 0) for s in seq], seq,
        softmax_scale=softmax_scale, k_scale=k_scale, v_scale=v_scale,
        causal=True, sliding_window=sliding_window,
    )


def extend(
    q: np.ndarray,
    k_pool: np.ndarray,
    v_pool: np.ndarray,
    req_to_token: np.ndarray,
    req_pool_indices: Sequence[int],
    prefix_lens: Sequence[int],
    extend_lens: Sequence[int],
    *,
    softmax_scale: float,
    k_scale: float = 1.0,
    v_scale: float = 1.0,
    causal: bool = True,
    sliding_window: int = -1,
) -> np.ndarray:
    """Prefix-aware extend: ``q`` [sum(E), Hq, D]; keys are prefix + extend of each sequence.

    The extend tokens' own K/V must already be in the pool (the backend writes
    them with ``set_kv_buffer`` before attending, flash_attn_v100_backend.py:1174-1182).
    """
    B = len(extend_lens)
    qsl = np.zeros(B + 1, dtype=np.int64)
    qsl[1:] = np.cumsum(np.asarray(extend_lens, dtype=np.int64))
    seq = [int(p) + int(e) for p, e in zip(prefix_lens, extend_lens)]
    slots = [slots_from_token_table(req_to_token, int(req_pool_indices[b]), seq[b]) for b in range(B)]
    return paged_attention(
        q, k_pool, v_pool, slots, qsl, prefix_lens, seq,
        softmax_scale=softmax_scale, k_scale=k_scale, v_scale=v_scale,
        causal=causal, sliding_window=sliding_window,
    )


def verify(
    q: np.ndarray,
    k_pool: np.ndarray,
    v_pool: np.ndarray,
    req_to_token: np.ndarray,
    req_pool_indices: Sequence[int],
    prefix_lens: Sequence[int],
    draft_token_num: int,
    **kw,
) -> np.ndarray:
    """Linear-chain target verify: extend with ``E = draft_token_num`` for every sequence."""
    return extend(q, k_pool, v_pool, req_to_token, req_pool_indices, prefix_lens,
                  [int(draft_token_num)] * len(prefix_lens), **kw)


def brute_force(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float,
                visible: Optional[np.ndarray] = None) -> np.ndarray:
    """Scalar loops for tiny shapes: q [R, D], k/v [n, D] -> [R, D] (zeros for an empty row)."""
    R, D = q.shape
    n = k.shape[0]
    out = np.zeros((R, v.shape[1]))
    for r in range(R):
        cols = [j for j in range(n) if visible is None or visible[r, j]]
        if not cols:
            continue
        s = [sum(q[r, d] * k[j, d] for d in range(D)) * scale for j in cols]
        mx = max(s)
        w = [np.exp(x - mx) for x in s]
        tot = sum(w)
        for c in range(v.shape[1]):
            out[r, c] = sum(wj * v[j, c] for wj, j in zip(w, cols)) / tot
    return out
