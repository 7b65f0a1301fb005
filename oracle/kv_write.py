"""The KV write into the token pool (``set_kv_buffer``), restated with numpy.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

The reference's backend writes each forward's new K/V through the pool's
``set_kv_buffer(layer, loc, k, v, k_scale, v_scale)``
(sglang_restomod/attention/v100/flash_attn_v100_backend.py:1174-1182, 1038-1046;
draft_decode.py:132-139). The pool is upstream SGLang's token pool: when the
cache dtype differs from the source dtype it divides the source by the scale *in
the source dtype* (``cache_k.div_(k_scale)``) and casts with torch
(``.to(cache dtype)``), storing fp8 as bytes; rows land at ``k_buffer[loc]``.

Restated here from the definitions:

* ``div16``: the quotient is computed in fp32 (correctly rounded) and rounded to
  the 16-bit source dtype (round to nearest even), which is what a bf16/fp16
  in-place division by a float does.
* ``to_fp8``: round to nearest, ties to the even code, on the grid of finite
  values of the format, with the first code past the largest finite value standing
  for overflow: e4m3fn has no infinity, so anything that rounds past 448 becomes
  NaN (0x7f / 0xff); e5m2 overflows to infinity (0x7c / 0xfc). NaN becomes 0x7f
  with its sign bit.
  This is OCP 8-bit floating point (v1.0) with the cast's overflow convention.

Pinned by ``tests/test_oracle_kv_write.py`` against torch's own division and cast
over every bf16 and every fp16 bit pattern at several scales.
"""

from __future__ import annotations

from typing import Optional

import numpy as np

from . import fp8 as F8

E4M3 = F8.E4M3
E5M2 = F8.E5M2


def _grid(fmt: str):
    """Non-negative finite values of the format, their codes, and the overflow code."""
    codes = np.arange(128, dtype=np.uint8)
    vals = F8.decode(codes, fmt)
    finite = np.isfinite(vals)
    codes, vals = codes[finite], vals[finite]
    order = np.argsort(vals, kind="stable")
    codes, vals = codes[order], vals[order]
    if fmt == E4M3:
        over_val, over_code = 480.0, 0x7F  # the code after 448 is the NaN pattern
    else:
        over_val, over_code = 65536.0, 0x7C  # infinity
    return np.append(vals, over_val), np.append(codes, over_code).astype(np.uint8), over_code


def to_fp8(x: np.ndarray, fmt: str) -> np.ndarray:
    """float values -> fp8 codes (uint8), round to nearest even code."""
    x = np.asarray(x, dtype=np.float64)
    vals, codes, over = _grid(fmt)
    a = np.abs(x)
    sign = (np.signbit(x)).astype(np.uint8) << 7
    hi = np.clip(np.searchsorted(vals, a, side="left"), 1, len(vals) - 1)
    lo = hi - 1
    dlo = a - vals[lo]
    dhi = vals[hi] - a
    pick_hi = (dhi < dlo) | ((dhi == dlo) & ((codes[hi] & 1) == 0) & ((codes[lo] & 1) == 1))
    idx = np.where(pick_hi, hi, lo)
    idx = np.where(a >= vals[-1], len(vals) - 1, idx)  # at or past the overflow value
    out = codes[idx] | sign
    out = np.where(a < vals[0] + 0.0, sign, out)  # (vals[0] is 0)
    out = np.where(np.isnan(x), np.uint8(0x7F) | sign, out)
    if fmt == E5M2:
        out = np.where(np.isinf(x), np.uint8(over) | sign, out)
    else:
        out = np.where(np.isinf(x), np.uint8(0x7F) | sign, out)
    return out.astype(np.uint8)


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint32) << 16).view(np.float32)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """Round fp32 to bf16 bits, nearest even; NaN stays NaN."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    r = np.where(nan, (u >> 16) | 0x40, r)
    return r.astype(np.uint16)


def f16_to_f32(bits: np.ndarray) -> np.ndarray:
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


def source_values(bits: np.ndarray, src: str) -> np.ndarray:
    return bf16_to_f32(bits) if src == "bf16" else f16_to_f32(bits)


def div16(bits: np.ndarray, src: str, scale: float) -> np.ndarray:
    """Source values divided by `scale` in fp32, rounded back to the source dtype (as fp32)."""
    with np.errstate(over="ignore", invalid="ignore", divide="ignore"):
        q = source_values(bits, src) / np.float32(scale)
        if src == "bf16":
            return bf16_to_f32(f32_to_bf16(q))
        return q.astype(np.float16).astype(np.float32)


def quantize(bits: np.ndarray, src: str, dst: str, scale: Optional[float]) -> np.ndarray:
    """Cache bytes (fp8) or 16-bit bits for source bits `bits` (uint16)."""
    bits = np.asarray(bits, dtype=np.uint16)
    if dst == src:
        return bits.copy()
    vals = div16(bits, src, scale) if scale is not None else source_values(bits, src)
    if dst in (E4M3, E5M2):
        with np.errstate(invalid="ignore"):
            return to_fp8(vals, dst)
    if dst == "bf16":
        return f32_to_bf16(vals)
    with np.errstate(over="ignore"):  # beyond fp16's range rounds to inf, as the kernel does
        return vals.astype(np.float16).view(np.uint16)


def set_kv_buffer(cache: np.ndarray, loc: np.ndarray, src_bits: np.ndarray, src: str, dst: str,
                  scale: Optional[float]) -> np.ndarray:
    """cache[loc[t]] = quantize(src_bits[t]) (slots distinct, as the engine allocates them)."""
    out = cache.copy()
    q = quantize(src_bits, src, dst, scale)
    for t, slot in enumerate(np.asarray(loc, dtype=np.int64)):
        out[slot] = q[t]
    return out
