"""Bit-level decoding of the two 8-bit KV formats (OCP e4m3fn and e5m2).

The reference dequantizes fp8 KV with torch's own cast: its 256-entry table is
``arange(256, uint8).view(fp8).to(fp16)`` (sglang_restomod/attention/v100/
tilelang/_paged_adapter.py:373-386), and e5m2 is additionally decoded with a
byte shift that the reference tests bitwise against that table
(tests/test_e5m2_shift_lut.py:19-33). Values are then scaled per tensor:
scores by ``softmax_scale * k_scale`` and outputs by ``v_scale``
(_paged_adapter.py:658, 753-754).

This module restates both formats from their published definitions (OCP 8-bit
floating point specification, v1.0):

* e4m3fn: 1 sign, 4 exponent (bias 7), 3 mantissa bits. Exponent 0 is
  subnormal (``m * 2**-9``). ``S.1111.111`` is NaN; there is no infinity.
* e5m2: 1 sign, 5 exponent (bias 15), 2 mantissa bits. Exponent 0 is subnormal
  (``m * 2**-16``). Exponent 31 is infinity (m = 0) or NaN (m != 0).

Pinned by ``tests/test_oracle_fp8.py``: all 256 codes of both formats against
torch's cast (a library routine), plus hand-computed known values (1.0, the
largest finite, the smallest subnormal, the NaN codes).
"""

from __future__ import annotations

import numpy as np

E4M3 = "e4m3fn"
E5M2 = "e5m2"


def decode_e4m3fn(raw: np.ndarray) -> np.ndarray:
    """Decode e4m3fn bytes to float64 (NaN for S.1111.111)."""
    b = np.asarray(raw, dtype=np.uint8).astype(np.int64)
    sign = np.where(b & 0x80, -1.0, 1.0)
    exp = (b >> 3) & 0xF
    man = b & 0x7
    normal = np.ldexp(1.0 + man / 8.0, exp - 7)
    subnormal = np.ldexp(man.astype(np.float64), -9)
    val = np.where(exp == 0, subnormal, normal) * sign
    return np.where((exp == 15) & (man == 7), np.nan, val)


def decode_e5m2(raw: np.ndarray) -> np.ndarray:
    """Decode e5m2 bytes to float64 (±inf for exponent 31 / mantissa 0)."""
    b = np.asarray(raw, dtype=np.uint8).astype(np.int64)
    sign = np.where(b & 0x80, -1.0, 1.0)
    exp = (b >> 2) & 0x1F
    man = b & 0x3
    normal = np.ldexp(1.0 + man / 4.0, exp - 15)
    subnormal = np.ldexp(man.astype(np.float64), -16)
    val = np.where(exp == 0, subnormal, normal) * sign
    val = np.where((exp == 31) & (man == 0), np.inf * sign, val)
    return np.where((exp == 31) & (man != 0), np.nan, val)


def decode(raw: np.ndarray, fmt: str) -> np.ndarray:
    if fmt == E4M3:
        return decode_e4m3fn(raw)
    if fmt == E5M2:
        return decode_e5m2(raw)
    raise ValueError(f"unknown fp8 format {fmt!r}")


def e5m2_to_f16_bits(raw: np.ndarray) -> np.ndarray:
    """The byte-shift decode the reference uses for e5m2 (``u16(raw) << 8``).

    _kernels_paged_decode.py:133-139. E5M2 and IEEE half share sign and
    exponent positions, so this is exact for every finite code.
    """
    return (np.asarray(raw, dtype=np.uint16) << 8).astype(np.uint16)
