"""Per-forward metadata restated with plain loops (small inputs only).

* ``page_table_from_indices`` follows
  sglang_restomod/attention/v100/draft_decode_plan.py:42-78: row ``r`` of a flat
  ``kv_indptr`` / ``kv_indices`` list has ``indptr[r+1] - indptr[r]`` tokens;
  logical page ``p`` is ``kv_indices[indptr[r] + p * ps] // ps`` while
  ``p * ps`` is inside the row, else 0; a buffer too short for the rows writes
  nothing and returns 0; an empty index list zeroes every row.
  Pinned by the reference's own known-answer vectors
  (tests/test_native_draft_decode_plan.py:22-87), restated in
  ``tests/test_oracle_metadata.py``.
* ``build_extend_metadata`` follows flash_attn_v100_backend.py:432-565:
  ``seq_lens = max(seq_lens, prefix + extend)`` (:452-455), page table
  ``req_to_token[req, 0:max_len:ps] // ps`` in a fixed-width zero-filled table
  (:465-490), ``query_start_loc = [0, cumsum(extend)]`` (:505-508), and the
  verify ("smallq") views: every query row repeats its sequence's page table
  and sees ``prefix + i + 1`` keys (:514-545).
  Pinned by hand-computed vectors in ``tests/test_oracle_metadata.py``.
* ``draft_rows`` restates the key rows of a multi-step draft round: row
  ``b * topk + k`` is request ``b``'s prefix ``req_to_token[req, :seq_b]`` followed by
  branch ``k``'s ``num_steps`` draft slots at ``req_to_token[req, seq_b + k * num_steps + s]``.
  The rule is the engine's placement of draft tokens at page size 1 (or top-k 1), which
  the reference's draft container consumes through the engine's per-step index builder
  (sglang_restomod/attention/v100/draft_decode.py:172-208; the builder itself is
  upstream SGLang 0.5.23, not in the reference). Pinned by the closed form at top-k 1
  (each row is the request's own ``req_to_token`` row), by the invariant that the
  branches' draft regions tile ``[seq_b, seq_b + topk * num_steps)`` without overlap,
  and by hand-computed vectors (``tests/test_oracle_metadata.py``). Against the engine's
  own builder it is parity unpinned (no vector of it exists in the reference).
"""

from __future__ import annotations

from typing import Dict, List, Sequence


def page_table_from_indices(kv_indptr: Sequence[int], kv_indices: Sequence[int],
                            rows_capacity: int, max_pages: int, page_size: int):
    """Return ``(rows, page_table, seq_lens)`` as lists (``rows == 0`` means nothing written)."""
    rows = len(kv_indptr) - 1
    if rows <= 0 or rows_capacity < rows:
        return 0, None, None
    table = [[0] * max_pages for _ in range(rows)]
    seq = [0] * rows
    if len(kv_indices) == 0:
        return rows, table, seq
    for r in range(rows):
        start, end = int(kv_indptr[r]), int(kv_indptr[r + 1])
        seq[r] = end - start
        for p in range(max_pages):
            off = p * page_size
            if off < end - start:
                idx = min(start + off, len(kv_indices) - 1)
                table[r][p] = int(kv_indices[idx]) // page_size
    return rows, table, seq


def build_extend_metadata(req_to_token: Sequence[Sequence[int]], req_pool_indices: Sequence[int],
                          seq_lens: Sequence[int], extend_seq_lens: Sequence[int],
                          extend_prefix_lens: Sequence[int], page_size: int, table_width: int,
                          build_smallq: bool = False) -> Dict[str, List]:
    B = len(seq_lens)
    seq = [max(int(s), int(p) + int(e)) for s, p, e in zip(seq_lens, extend_prefix_lens, extend_seq_lens)]
    max_len = max(seq) if B else 0
    max_pages = (max_len + page_size - 1) // page_size
    table = [[0] * table_width for _ in range(B)]
    for b in range(B):
        row = req_to_token[int(req_pool_indices[b])]
        for p in range(max_pages):
            table[b][p] = int(row[p * page_size]) // page_size
    qsl = [0]
    for e in extend_seq_lens:
        qsl.append(qsl[-1] + int(e))
    md = {
        "page_table": table,
        "seq_lens": seq,
        "query_start_loc": qsl,
        "prefix_kv_lens": [int(p) for p in extend_prefix_lens],
        "max_seq_len": max_len,
    }
    if build_smallq:
        sq_table, sq_seq = [], []
        for b in range(B):
            for i in range(int(extend_seq_lens[b])):
                sq_table.append(list(table[b]))
                sq_seq.append(int(extend_prefix_lens[b]) + i + 1)
        md["smallq_page_table"] = sq_table
        md["smallq_seq_lens"] = sq_seq
    return md


def draft_rows(req_to_token: Sequence[Sequence[int]], req_pool_indices: Sequence[int], seq_lens: Sequence[int],
               topk: int, num_steps: int, mapping: Sequence[int] | None = None) -> List[List[int]]:
    """Rows ``b * topk + k``: prefix slots, then branch ``k``'s ``num_steps`` draft slots
    (positions past the table's width read as slot 0; ``mapping`` translates every slot,
    one outside it giving 0)."""
    def at(row, p):
        slot = int(row[p]) if p < len(row) else 0
        if mapping is not None:
            slot = int(mapping[slot]) if 0 <= slot < len(mapping) else 0
        return slot

    out = []
    for b, seq in enumerate(seq_lens):
        row = req_to_token[int(req_pool_indices[b])]
        seq = max(int(seq), 0)
        for k in range(topk):
            out.append([at(row, j) for j in range(seq)] +
                       [at(row, seq + k * num_steps + s) for s in range(num_steps)])
    return out
