"""Pins oracle/metadata.py with the reference's own known-answer vectors
(tests/test_native_draft_decode_plan.py:22-87) and hand-computed extend metadata."""

from oracle import metadata as M


def test_page_table_reads_the_page_start_of_each_row():
    row0 = [0, 1, 2, 3, 12, 13, 14, 15, 8]
    row1 = [20, 21, 22, 23, 4]
    rows, table, seq = M.page_table_from_indices([0, 9, 14], row0 + row1, 2, 3, 4)
    assert rows == 2 and seq == [9, 5] and table == [[0, 3, 2], [5, 1, 0]]


def test_page_table_marks_unused_pages_zero():
    rows, table, seq = M.page_table_from_indices([0, 4, 4], list(range(32)), 2, 2, 4)
    assert seq == [4, 0] and table == [[0, 0], [0, 0]]


def test_page_table_handles_an_empty_index_list():
    rows, table, seq = M.page_table_from_indices([0, 1], [], 1, 2, 4)
    assert rows == 1 and seq == [0] and table == [[0, 0]]


def test_page_table_refuses_a_short_buffer():
    assert M.page_table_from_indices([0, 4, 8], list(range(8)), 1, 1, 16)[0] == 0


def test_extend_metadata_by_hand():
    # two requests in rows 2 and 0 of req_to_token, page size 2
    r2t = [[10, 11, 4, 5, 0, 0], [0] * 6, [6, 7, 2, 3, 8, 9]]
    md = M.build_extend_metadata(r2t, [2, 0], seq_lens=[1, 1], extend_seq_lens=[2, 1],
                                 extend_prefix_lens=[3, 2], page_size=2, table_width=4, build_smallq=True)
    assert md["seq_lens"] == [5, 3]                      # max(seq, prefix + extend)
    assert md["page_table"] == [[3, 1, 4, 0], [5, 2, 0, 0]]
    assert md["query_start_loc"] == [0, 2, 3]
    assert md["prefix_kv_lens"] == [3, 2]
    assert md["smallq_seq_lens"] == [4, 5, 3]            # prefix + i + 1
    assert md["smallq_page_table"] == [[3, 1, 4, 0], [3, 1, 4, 0], [5, 2, 0, 0]]


def test_draft_rows_by_hand():
    # request row 1: prefix of 3 tokens, then 2 branches x 2 steps of draft slots
    r2t = [[0] * 9, [40, 41, 42, 50, 51, 60, 61, 0, 0]]
    rows = M.draft_rows(r2t, [1], [3], topk=2, num_steps=2)
    assert rows == [[40, 41, 42, 50, 51], [40, 41, 42, 60, 61]]
    # through a mapping, with a slot outside it giving 0
    rows = M.draft_rows(r2t, [1], [3], topk=1, num_steps=2, mapping=list(range(100, 152)))
    assert rows == [[140, 141, 142, 150, 151]]
    rows = M.draft_rows(r2t, [1], [3], topk=2, num_steps=2, mapping=list(range(100, 152)))
    assert rows[1] == [140, 141, 142, 0, 0]  # slots 60 and 61 lie outside the mapping


def test_draft_rows_top1_is_the_request_row():
    import random

    rnd = random.Random(3)
    r2t = [[rnd.randrange(1, 1000) for _ in range(64)] for _ in range(5)]
    for req, seq, steps in ((4, 10, 3), (0, 1, 5), (2, 40, 1), (3, 0, 2)):
        assert M.draft_rows(r2t, [req], [seq], topk=1, num_steps=steps) == [r2t[req][:seq + steps]]


def test_draft_rows_branches_tile_the_draft_region():
    r2t = [list(range(1000, 1064))]
    seq, topk, steps = 7, 4, 3
    rows = M.draft_rows(r2t, [0], [seq], topk=topk, num_steps=steps)
    tails = [r[seq:] for r in rows]
    flat = [s for t in tails for s in t]
    assert sorted(flat) == r2t[0][seq:seq + topk * steps]  # disjoint, and they cover the region
    assert all(r[:seq] == r2t[0][:seq] for r in rows)      # every branch shares the prefix
