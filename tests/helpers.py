"""Shared test helpers."""

from __future__ import annotations

import numpy as np
import torch

# Tolerance for fp16/bf16 outputs against the float64 oracle: 2e-3 absolute on the
# softmax-normalised output, plus half an ulp of the reference value in the output
# dtype, because the output itself is stored in that dtype (an exact result rounded
# to bf16 is already up to half an ulp away).
ATOL = 2e-3


def half_ulp(ref: np.ndarray, dtype: torch.dtype) -> np.ndarray:
    mant = 7 if dtype == torch.bfloat16 else 10
    mag = np.maximum(np.abs(ref), 2.0 ** -14)
    return 0.5 * np.exp2(np.floor(np.log2(mag)) - mant)


def assert_attn_close(out: torch.Tensor, ref: np.ndarray, atol: float = ATOL, what: str = "") -> float:
    got = out.detach().float().cpu().numpy().astype(np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    err = np.abs(got - ref)
    bound = atol + half_ulp(ref, out.dtype)
    bad = err > bound
    if bad.any():
        idx = np.unravel_index(np.argmax(err - bound), err.shape)
        raise AssertionError(
            f"{what}: {int(bad.sum())} of {err.size} elements exceed {atol} + half-ulp; "
            f"worst at {idx}: got {got[idx]:.6f} want {ref[idx]:.6f} (err {err[idx]:.3e})"
        )
    return float(err.max())


def to_f64(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy().astype(np.float64)


def pool_f64(pool: torch.Tensor, scale: float = 1.0) -> np.ndarray:
    """Dequantize a KV pool to float64 with torch's own cast (``raw.float() * scale``)."""
    return pool.detach().cpu().float().numpy().astype(np.float64) * scale
