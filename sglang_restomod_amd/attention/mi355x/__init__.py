"""MI355X attention component.

Registers ``MI355XAttnBackend`` with the engine's attention registry under
``mi355x_attn`` (and, when ``SGLANG_MI355X_ATTN_ALIAS_V100=1``, also under the
V100 backend's name ``tilelang_fa_v100`` so an existing launch profile switches
without edits). Mirrors sglang_restomod/attention/v100/__init__.py:18-34.

Selection: ``SGLANG_RESTOMOD_COMPONENTS=attention_mi355x``.
"""

from __future__ import annotations


def register() -> None:
    """Component entry point: register the backend name(s), the draft choice, and the
    draft factory hook."""
    from . import draft_backend
    from .backend_registry import install, install_draft_choices

    install()
    install_draft_choices()
    draft_backend.install()
