"""The HIP kernels against the committed golden fixtures (tests/golden/*.npz).

Decode fixtures run through ma_grouped_decode; extend and verify fixtures run
through both ma_paged_extend and ma_paged_verify, which must each match.
"""

from __future__ import annotations

import pytest
import torch

from tests import golden_io
from tests.helpers import assert_attn_close

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def _ops():
    from sglang_restomod_amd.attention.mi355x import ops

    return ops


def _device_case(name):
    c = golden_io.load(name)
    d = {k: c[k + "_t"].to(DEV) for k in ("q", "k", "v")}
    d["r2t"] = torch.from_numpy(c["req_to_token"]).to(DEV)
    d["rpi"] = torch.from_numpy(c["req_pool_indices"]).to(DEV)
    d["seq"] = torch.from_numpy(c["seq_lens"]).to(DEV)
    d["pre"] = torch.from_numpy(c["prefix_lens"]).to(DEV)
    d["qsl"] = torch.from_numpy(c["query_start_loc"]).to(DEV)
    return c, d


def _scales(c):
    return dict(softmax_scale=float(c["softmax_scale"]), k_scale=float(c["k_scale"]), v_scale=float(c["v_scale"]))


@pytest.mark.parametrize("name", [n for n in golden_io.names() if n.startswith("decode")])
def test_decode_matches_fixture(name):
    c, d = _device_case(name)
    out = _ops().grouped_decode_forward(d["q"], d["k"], d["v"], d["r2t"], d["seq"], row_index=d["rpi"],
                                        sliding_window_size=int(c["window"]), **_scales(c))
    torch.cuda.synchronize()
    assert_attn_close(out, c["expected"], what=name)


@pytest.mark.parametrize("kernel", ["extend", "verify"])
@pytest.mark.parametrize("name", [n for n in golden_io.names() if not n.startswith("decode")])
def test_extend_and_verify_match_fixture(name, kernel):
    c, d = _device_case(name)
    qlens = (c["query_start_loc"][1:] - c["query_start_loc"][:-1]).tolist()
    common = dict(causal=bool(c["causal"]), sliding_window_size=int(c["window"]), row_index=d["rpi"], **_scales(c))
    ops = _ops()
    if kernel == "extend":
        out = ops.paged_extend_forward(d["q"], d["k"], d["v"], d["r2t"], d["seq"], d["qsl"], d["pre"],
                                       **common)
    else:
        out = ops.paged_verify_forward(d["q"], d["k"], d["v"], d["r2t"], d["seq"], d["qsl"], d["pre"],
                                       max_q_per_seq=max(qlens), **common)
    torch.cuda.synchronize()
    assert_attn_close(out, c["expected"], what=f"{name} via {kernel}")
