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
