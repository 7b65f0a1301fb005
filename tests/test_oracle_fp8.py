"""Pins oracle/fp8.py: every byte of both formats against torch's cast, plus known values."""

import numpy as np
import pytest
import torch

from oracle import fp8


@pytest.mark.parametrize("fmt,tdt", [(fp8.E4M3, torch.float8_e4m3fn), (fp8.E5M2, torch.float8_e5m2)])
def test_all_256_codes_match_torch(fmt, tdt):
    raw = np.arange(256, dtype=np.uint8)
    ours = fp8.decode(raw, fmt)
    theirs = torch.from_numpy(raw).view(tdt).to(torch.float64).numpy()
    nan = np.isnan(theirs)
    assert (np.isnan(ours) == nan).all()
    assert np.array_equal(ours[~nan], theirs[~nan])


def test_known_e4m3_values():
    d = lambda b: float(fp8.decode_e4m3fn(np.array([b], dtype=np.uint8))[0])
    assert d(0x38) == 1.0           # exponent 7 = bias
    assert d(0x7E) == 448.0         # largest finite
    assert d(0x01) == 2.0 ** -9     # smallest subnormal
    assert d(0x08) == 2.0 ** -6     # smallest normal
    assert d(0xB8) == -1.0
    assert np.isnan(d(0x7F)) and np.isnan(d(0xFF))


def test_known_e5m2_values():
    d = lambda b: float(fp8.decode_e5m2(np.array([b], dtype=np.uint8))[0])
    assert d(0x3C) == 1.0
    assert d(0x7B) == 57344.0
    assert d(0x01) == 2.0 ** -16
    assert d(0x7C) == np.inf and d(0xFC) == -np.inf
    assert np.isnan(d(0x7D))


def test_e5m2_shift_reproduces_torch_for_finite_bytes():
    """The reference's e5m2 shift (tests/test_e5m2_shift_lut.py:19-33), restated."""
    raw = np.arange(256, dtype=np.uint8)
    lut = torch.from_numpy(raw).view(torch.float8_e5m2).to(torch.float16)
    shifted = torch.from_numpy(fp8.e5m2_to_f16_bits(raw).view(np.int16)).view(torch.float16)
    finite = ~torch.isnan(lut)
    assert torch.equal(lut.view(torch.int16)[finite], shifted.view(torch.int16)[finite])
    assert torch.isnan(shifted[~finite]).all()


def test_a_wrong_bias_would_fail():
    """Sanity: the pin detects a plausible mistake (e4m3 decoded with the e5m2 bias)."""
    raw = np.arange(256, dtype=np.uint8)
    wrong = fp8.decode_e5m2(raw)
    theirs = torch.from_numpy(raw).view(torch.float8_e4m3fn).to(torch.float64).numpy()
    ok = ~np.isnan(theirs) & ~np.isnan(wrong)
    assert not np.array_equal(wrong[ok], theirs[ok])
