"""Load the committed golden fixtures (tests/golden/*.npz) as tensors / float64 arrays."""

from __future__ import annotations

import glob
import os

import numpy as np
import torch

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TORCH = {"bf16": torch.bfloat16, "fp16": torch.float16, "e4m3": torch.float8_e4m3fn, "e5m2": torch.float8_e5m2}


def names():
    return sorted(os.path.basename(p)[:-4] for p in glob.glob(os.path.join(GOLDEN, "*.npz")))


def _tensor(bits: np.ndarray, dt: str) -> torch.Tensor:
    t = torch.from_numpy(bits.copy())
    if dt in ("bf16", "fp16"):
        return t.view(torch.int16).view(TORCH[dt])
    return t.view(TORCH[dt])


def load(name: str) -> dict:
    z = np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False)
    case = {k: z[k] for k in z.files}
    case["name"] = name
    case["q_t"] = _tensor(case["q"], str(case["q_dtype"]))
    case["k_t"] = _tensor(case["k"], str(case["kv_dtype"]))
    case["v_t"] = _tensor(case["v"], str(case["kv_dtype"]))
    return case


def f64(t: torch.Tensor) -> np.ndarray:
    return t.float().numpy().astype(np.float64)
