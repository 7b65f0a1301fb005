"""Attestation record: which components of this plugin registered, for an outside verifier.

The record is a JSON object with these keys (the interface the reference's verifier
reads; format of sglang_restomod/attest.py:138-194):

``engine``
    ``{"python": version, "path": module file or null, "version": or null}`` of the
    ``sglang`` module as imported in this process (null when it is not imported).
``selected``
    the component names the environment selected, in order.
``components``
    ``{name: {"ok": bool, "detail": text}}``; ``detail`` is present only when there is
    one. An inactive component's detail starts with ``"registered, inactive: "``.
``loaded`` / ``failed`` / ``inactive``
    names by outcome, in the order the outcomes were first reported. ``inactive`` is a
    subset of ``loaded`` (the component registered without error but serves nothing).
``missing``
    selected names with no outcome at all.

Design: one ``_Outcome`` per component in an insertion-ordered table; the lists are
derived from it when a snapshot is taken, so they cannot disagree. ``write`` renders
the snapshot into a uniquely named sibling file and renames it over the target, so
concurrent writers (one per rank) never share a partial file. Nothing here raises into
the caller: attestation is an observer and must not stop a launch.
"""

from __future__ import annotations

import json
import logging
import os
import secrets
import sys
from dataclasses import dataclass
from typing import Any, Optional

logger = logging.getLogger(__name__)

ENV_ATTEST = "SGLANG_RESTOMOD_ATTEST"
INACTIVE_PREFIX = "registered, inactive: "


@dataclass
class _Outcome:
    ok: bool
    detail: str = ""
    idle: bool = False  # registered, but serves nothing

    def as_json(self) -> dict[str, Any]:
        out: dict[str, Any] = {"ok": self.ok}
        if self.detail:
            out["detail"] = self.detail
        return out


class _Ledger:
    def __init__(self) -> None:
        self.selected: list[str] = []
        self.outcomes: dict[str, _Outcome] = {}

    def names(self, pred) -> list[str]:
        return [name for name, o in self.outcomes.items() if pred(o)]


_LEDGER = _Ledger()


def reset() -> None:
    """Forget every outcome and the selection (tests)."""
    global _LEDGER
    _LEDGER = _Ledger()


def set_selected(names: list[str]) -> None:
    _LEDGER.selected = [str(n) for n in names]


def record(name: str, ok: bool, detail: str = "") -> None:
    """Report one component's registration: ``ok`` True for a clean ``register()``, False
    for one that raised. A success without a detail keeps what an earlier report said
    (an inactive reason survives the later success report); a failure ends any inactive
    state."""
    prev = _LEDGER.outcomes.get(name)
    if ok:
        idle = prev.idle if prev is not None else False
        text = detail or (prev.detail if prev is not None else "")
        _LEDGER.outcomes[name] = _Outcome(True, text, idle)
    else:
        _LEDGER.outcomes[name] = _Outcome(False, detail, False)


def inactive(name: str, reason: Any) -> None:
    """Report a component that registered (or was selected) but serves nothing."""
    try:
        text = f"{reason}"
    except Exception:  # noqa: BLE001 - a reason that cannot print is still a reason
        text = "<reason could not be printed>"
    _LEDGER.outcomes[name] = _Outcome(True, INACTIVE_PREFIX + text, True)


def engine() -> dict[str, Any]:
    """Identity of the engine as this process imported it (not as some installer put it)."""
    module = sys.modules.get("sglang")
    return {
        "python": sys.version.split()[0],
        "path": None if module is None else getattr(module, "__file__", None),
        "version": None if module is None else getattr(module, "__version__", None),
    }


def snapshot() -> dict[str, Any]:
    led = _LEDGER
    return {
        "engine": engine(),
        "selected": list(led.selected),
        "components": {name: o.as_json() for name, o in led.outcomes.items()},
        "loaded": led.names(lambda o: o.ok),
        "failed": led.names(lambda o: not o.ok),
        "inactive": led.names(lambda o: o.idle),
        "missing": [n for n in led.selected if n not in led.outcomes],
    }


def write(path: Optional[str] = None) -> Optional[str]:
    """Write the snapshot to ``path`` (default: ``$SGLANG_RESTOMOD_ATTEST``). Returns the
    path written, or None when no target is set or the write failed."""
    target = path if path else os.environ.get(ENV_ATTEST, "")
    if not target:
        return None
    staging = f"{target}.{os.getpid()}.{secrets.token_hex(4)}.part"
    try:
        text = json.dumps(snapshot(), indent=2, sort_keys=True) + "\n"
        with open(staging, "x", encoding="utf-8") as fh:  # "x": never reuse another writer's file
            fh.write(text)
        os.replace(staging, target)
        return target
    except Exception:  # noqa: BLE001 - report, never raise into the engine's startup
        logger.warning("attestation not written to %s", target, exc_info=True)
        try:
            os.unlink(staging)
        except OSError:
            pass
        return None
