"""Component registry (same contract as sglang_restomod/plugins.py:26-194).

* ``SGLANG_RESTOMOD_COMPONENTS`` is a comma-separated list of component names;
  blanks are ignored and duplicates dropped in first-seen order (:107-114).
* An unknown name raises ``ValueError`` listing the known ones (:115-122).
* ``load_enabled`` imports each selected component and calls its
  ``register()``. Nothing raises out of it: an import failure or a module
  without ``register`` is recorded as inactive, a ``register()`` that raises is
  recorded as failed, and the remaining components still load (:129-194).

Importing this module pulls in neither torch nor any kernel.
"""

from __future__ import annotations

import importlib
import logging
import os
from collections.abc import Mapping, Sequence
from dataclasses import dataclass

logger = logging.getLogger(__name__)

ENV_COMPONENTS = "SGLANG_RESTOMOD_COMPONENTS"


@dataclass(frozen=True)
class Component:
    name: str
    module: str
    description: str


COMPONENTS: dict[str, Component] = {
    "attention_mi355x": Component(
        name="attention_mi355x",
        module="sglang_restomod_amd.attention.mi355x",
        description="MI355X paged attention backend: split-KV decode, prefix-aware extend, "
        "linear-chain target verify, fp8 KV; hand-written gfx950 HIP kernels",
    ),
}


def selection(env: Mapping[str, str] | None = None) -> list[str]:
    """Selected component names, validated, de-duplicated, in order."""
    source = os.environ if env is None else env
    names: list[str] = []
    for part in source.get(ENV_COMPONENTS, "").split(","):
        name = part.strip()
        if name and name not in names:
            names.append(name)
    unknown = [n for n in names if n not in COMPONENTS]
    if unknown:
        raise ValueError(
            f"unknown component(s) in {ENV_COMPONENTS}: {', '.join(unknown)}; "
            f"known: {', '.join(sorted(COMPONENTS))}"
        )
    return names


def is_enabled(name: str, env: Mapping[str, str] | None = None) -> bool:
    return name in selection(env)


def load_enabled(env: Mapping[str, str] | None = None) -> Sequence[str]:
    """Import and register each selected component; return the names that registered."""
    from . import attest

    names = selection(env)
    attest.set_selected(names)
    loaded: list[str] = []
    for name in names:
        comp = COMPONENTS[name]
        try:
            module = importlib.import_module(comp.module)
        except Exception as exc:  # noqa: BLE001 - recorded, the rest still load
            attest.inactive(name, f"import failed: {type(exc).__name__}: {exc}")
            logger.warning("component %s failed to import", name, exc_info=True)
            continue
        reg = getattr(module, "register", None)
        if reg is None:
            attest.inactive(name, f"imported {comp.module} but it has no register()")
            logger.warning("component %s has no register()", name)
            continue
        try:
            reg()
        except Exception as exc:  # noqa: BLE001
            attest.record(name, False, f"{type(exc).__name__}: {exc}")
            logger.warning("component %s failed to register", name, exc_info=True)
            continue
        attest.record(name, True)
        loaded.append(name)
    seen = attest.snapshot()["components"]
    for name in names:
        if name not in seen:
            attest.inactive(name, "selected but never registered")
    logger.info("%d/%d components active (%s)", len(loaded), len(names), ", ".join(loaded) or "none")
    return loaded
