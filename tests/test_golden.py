"""The float64 oracle against the committed golden fixtures (scalar brute-force
outputs, tests/golden/make_golden.py) and the fixtures' own consistency."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import attention as oracle
from tests import golden_io


def test_every_fixture_is_present():
    assert len(golden_io.names()) >= 11
    kinds = {n.split("_")[0] for n in golden_io.names()}
    assert kinds == {"decode", "extend", "verify"}


@pytest.mark.parametrize("name", golden_io.names())
def test_oracle_matches_fixture(name):
    c = golden_io.load(name)
    B = len(c["seq_lens"])
    seq = c["seq_lens"].tolist()
    slots = [oracle.slots_from_token_table(c["req_to_token"], int(c["req_pool_indices"][b]), seq[b])
             for b in range(B)]
    qsl = c["query_start_loc"].tolist()
    # decode rows see every key below seq_len: prefix = seq_len - 1
    prefix = [max(s - 1, 0) for s in seq] if name.startswith("decode") else c["prefix_lens"].tolist()
    got = oracle.paged_attention(
        golden_io.f64(c["q_t"]), golden_io.f64(c["k_t"]), golden_io.f64(c["v_t"]), slots, qsl, prefix, seq,
        softmax_scale=float(c["softmax_scale"]), k_scale=float(c["k_scale"]), v_scale=float(c["v_scale"]),
        causal=bool(c["causal"]), sliding_window=int(c["window"]))
    np.testing.assert_allclose(got, c["expected"], rtol=1e-10, atol=1e-12)


def test_fixture_tables_are_consistent():
    for name in golden_io.names():
        c = golden_io.load(name)
        r2t, rpi, seq = c["req_to_token"], c["req_pool_indices"], c["seq_lens"]
        used = np.concatenate([r2t[rpi[b], :seq[b]] for b in range(len(seq))])
        assert len(set(used.tolist())) == used.size, name  # no slot is shared
        assert used.size == 0 or used.min() >= 1, name  # slot 0 is padding
        assert c["q_t"].shape[0] == c["query_start_loc"][-1], name
