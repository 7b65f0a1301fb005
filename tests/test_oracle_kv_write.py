"""The KV-write oracle against torch's own division and fp8 cast, exhaustively over
the 16-bit inputs (the upstream pool's ``k.div_(k_scale)`` then ``.to(fp8)``)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import kv_write as KW

SRC = {"bf16": torch.bfloat16, "fp16": torch.float16}
DST = {KW.E4M3: torch.float8_e4m3fn, KW.E5M2: torch.float8_e5m2}
ALL16 = np.arange(65536, dtype=np.uint32).astype(np.uint16)


def _torch_quantize(bits, src, dst, scale):
    t = torch.from_numpy(bits.astype(np.int16)).view(SRC[src])
    if scale is not None:
        t = t / scale
    return t.to(DST[dst]).view(torch.uint8).numpy()


def _is_nan_code(codes, dst):
    if dst == KW.E4M3:
        return (codes & 0x7F) == 0x7F
    return (codes & 0x7F) > 0x7C


@pytest.mark.parametrize("src", ["bf16", "fp16"])
@pytest.mark.parametrize("dst", [KW.E4M3, KW.E5M2])
@pytest.mark.parametrize("scale", [None, 1.0, 0.37, 2.5, 0.001, 3e4])
def test_every_16bit_input_matches_torch(src, dst, scale):
    """Bit-exact for every non-NaN input; a NaN input gives a NaN code (torch's CPU bf16
    arithmetic returns NaN with the sign bit set, its GPU arithmetic without)."""
    want = _torch_quantize(ALL16, src, dst, scale)
    got = KW.quantize(ALL16, src, dst, scale)
    nan_in = np.isnan(KW.source_values(ALL16, src))
    bad = np.nonzero((got != want) & ~nan_in)[0]
    assert bad.size == 0, [(hex(int(ALL16[i])), hex(int(got[i])), hex(int(want[i]))) for i in bad[:8]]
    assert _is_nan_code(got[nan_in], dst).all() and _is_nan_code(want[nan_in], dst).all()


def test_overflow_conventions():
    x = np.array([448.0, 463.99, 464.0, 479.0, 480.0, 1e9, np.inf, -np.inf, np.nan, -448.0])
    assert [hex(v) for v in KW.to_fp8(x, KW.E4M3)] == [
        "0x7e", "0x7e", "0x7e", "0x7f", "0x7f", "0x7f", "0x7f", "0xff", "0x7f", "0xfe"]
    y = np.array([57344.0, 61439.0, 61440.0, np.inf, -np.inf, np.nan])
    assert [hex(v) for v in KW.to_fp8(y, KW.E5M2)] == ["0x7b", "0x7b", "0x7c", "0x7c", "0xfc", "0x7f"]
    assert hex(KW.to_fp8(np.array([-np.nan]), KW.E4M3)[0]) == "0xff"


def test_a_truncating_cast_would_fail():
    # 1 + 3/16 lies between e4m3's 1.125 and 1.25 at a tie; even code is 1.25 (mantissa 010)
    assert hex(KW.to_fp8(np.array([1.1875]), KW.E4M3)[0]) == "0x3a"
    assert hex(KW.to_fp8(np.array([1.0625]), KW.E4M3)[0]) == "0x38"  # tie to even: 1.0


def test_same_dtype_is_a_copy_and_scatter_places_rows():
    bits = np.array([[1, 2], [3, 4], [5, 6]], dtype=np.uint16)
    cache = np.zeros((8, 2), dtype=np.uint16)
    out = KW.set_kv_buffer(cache, np.array([5, 0, 7]), bits, "bf16", "bf16", None)
    assert out[5].tolist() == [1, 2] and out[0].tolist() == [3, 4] and out[7].tolist() == [5, 6]
    assert out[1:5].sum() == 0
