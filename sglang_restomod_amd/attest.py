"""What actually registered, in a form a verifier can read (sglang_restomod/attest.py:1-194).

Three states per component:

* loaded (``record(name, True)``): registered and in use;
* failed (``record(name, False, detail)``): its ``register()`` raised;
* inactive (``inactive(name, reason)``): loaded cleanly but does nothing; it is
  also listed as loaded so the two lists stay a partition of "registered".

``snapshot()`` returns the record plus the imported engine's identity, and
lists as ``missing`` any selected name with no record. ``write()`` dumps the
snapshot as JSON to ``SGLANG_RESTOMOD_ATTEST`` (or a given path) through a
per-call temporary file and an atomic rename, so several ranks writing the same
target do not trip over one shared temporary name. No function here raises.
"""

from __future__ import annotations

import json
import logging
import os
import sys
import tempfile
from typing import Any

logger = logging.getLogger(__name__)

ENV_ATTEST = "SGLANG_RESTOMOD_ATTEST"


def _empty() -> dict[str, Any]:
    return {"selected": [], "components": {}, "loaded": [], "failed": [], "inactive": []}


_STATE: dict[str, Any] = _empty()


def reset() -> None:
    """Forget everything (tests)."""
    _STATE.clear()
    _STATE.update(_empty())


def set_selected(names: list[str]) -> None:
    _STATE["selected"] = list(names)


def engine() -> dict[str, Any]:
    """The engine as imported (module path and its own ``__version__``), not as installed."""
    mod = sys.modules.get("sglang")
    return {
        "python": sys.version.split()[0],
        "path": getattr(mod, "__file__", None) if mod is not None else None,
        "version": getattr(mod, "__version__", None) if mod is not None else None,
    }


def _add(key: str, name: str) -> None:
    if name not in _STATE[key]:
        _STATE[key].append(name)


def _drop(key: str, name: str) -> None:
    if name in _STATE[key]:
        _STATE[key].remove(name)


def record(name: str, ok: bool, detail: str = "") -> None:
    """One component's registration outcome; keeps an earlier inactive reason if none is given."""
    entry: dict[str, Any] = {"ok": bool(ok)}
    previous = _STATE["components"].get(name) or {}
    if detail:
        entry["detail"] = detail
    elif previous.get("detail"):
        entry["detail"] = previous["detail"]
    _STATE["components"][name] = entry
    if ok:
        _add("loaded", name)
        _drop("failed", name)
    else:
        _add("failed", name)


def inactive(name: str, reason: Any) -> None:
    """A component that registered (or was selected) but will do nothing. Never raises."""
    try:
        text = str(reason)
    except Exception:  # noqa: BLE001
        text = "<unprintable reason>"
    try:
        entry = _STATE["components"].setdefault(name, {"ok": True})
        entry["detail"] = "registered, inactive: " + text
        _add("inactive", name)
        _drop("failed", name)
        _add("loaded", name)
    except Exception:  # noqa: BLE001
        logger.debug("attest.inactive(%s) failed", name, exc_info=True)


def snapshot() -> dict[str, Any]:
    snap = {
        "engine": engine(),
        "selected": list(_STATE["selected"]),
        "loaded": list(_STATE["loaded"]),
        "failed": list(_STATE["failed"]),
        "inactive": list(_STATE["inactive"]),
        "components": {k: dict(v) for k, v in _STATE["components"].items()},
    }
    snap["missing"] = [n for n in snap["selected"] if n not in snap["components"]]
    return snap


def write(path: str | None = None) -> str | None:
    """Write the snapshot as JSON; return the path written or None (unset or unwritable)."""
    target = path or os.environ.get(ENV_ATTEST)
    if not target:
        return None
    tmp = None
    try:
        payload = snapshot()
        folder = os.path.dirname(target) or "."
        fd, tmp = tempfile.mkstemp(dir=folder, prefix=os.path.basename(target) + ".", suffix=".tmp")
        with os.fdopen(fd, "w", encoding="utf-8") as fh:
            json.dump(payload, fh, indent=1, sort_keys=True)
            fh.write("\n")
        os.replace(tmp, target)
        tmp = None
    except Exception:  # noqa: BLE001 - an observer's file never stops a launch
        logger.warning("could not write attestation to %s", target, exc_info=True)
        if tmp is not None:
            try:
                os.remove(tmp)
            except OSError:
                pass
        return None
    return target
