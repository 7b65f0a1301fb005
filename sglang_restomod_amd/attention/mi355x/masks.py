"""Per-layer mask decision (sglang_restomod/attention/v100/masks.py:13-35).

The kernels take a boolean ``causal`` and an integer window where ``-1`` means
none. A layer is causal when the engine's default says so and it is neither
cross-attention nor encoder-only. A window is kept for non-causal layers too:
the kernels apply it as a left bound only (keys from ``q - window`` on), which is
what a bidirectional sliding draft block needs. Torch-free on purpose.
"""

from __future__ import annotations

from typing import Optional


def resolve_layer_mask(
    *,
    default_causal: bool,
    is_cross_attention: bool,
    is_encoder_only: bool,
    sliding_window_size: Optional[int],
) -> tuple[bool, int]:
    causal = bool(default_causal) and not (bool(is_cross_attention) or bool(is_encoder_only))
    if sliding_window_size is None or int(sliding_window_size) < 0:
        return causal, -1
    return causal, int(sliding_window_size)
