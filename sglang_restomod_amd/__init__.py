"""MI355X-native attention hot path for SGLang, packaged as a restomod-style plugin.

SGLang discovers plugins through the ``sglang.srt.plugins`` entry-point group;
``register`` is the function that group names (sglang_restomod/__init__.py:24,
pyproject.toml:37-38 of the reference). Selection is one environment variable:

    SGLANG_RESTOMOD_COMPONENTS=attention_mi355x

With the variable unset the plugin loads and does nothing. Importing this
package is cheap: no torch, no kernels. The HIP library is loaded on first use
by the backend.
"""

from __future__ import annotations

import logging

__version__ = "0.1.0"

logger = logging.getLogger(__name__)


def register() -> None:
    """Entry point: load the selected components and write the attestation record."""
    from . import attest
    from .plugins import load_enabled, selection

    names = selection()
    if not names:
        # "loaded with nothing selected" is recorded, so it can be told apart
        # from "never ran".
        attest.set_selected([])
        attest.write()
        logger.info("sglang-restomod-amd: plugin loaded, no component selected")
        return
    loaded = load_enabled()
    logger.info("sglang-restomod-amd: plugin loaded (components: %s)", ", ".join(loaded) or "none")
    attest.write()
