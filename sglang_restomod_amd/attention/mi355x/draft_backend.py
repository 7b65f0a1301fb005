"""Let a draft worker select this backend (the role of
sglang_restomod/attention/v100/draft_backend.py:31-83).

The engine builds a draft worker's attention from a fixed name table in its
``DraftBackendFactory``. ``install_on`` reroutes two of the factory's methods by the
selected name: when it is one of ``NAMES``,

* ``create_draft_extend_backend`` returns ``MI355XAttnBackend`` inside the engine's
  draft-extend wrapper (a draft extend is a few rows per request over the whole
  prefix, which the backend serves with its split-KV verify kernel);
* ``create_decode_backend`` returns the split-KV multi-step container of
  ``draft_decode`` for drafts of two or more steps. A draft worker it cannot serve
  raises ``NotImplementedError`` from the container; nothing is handed to another
  backend.

Every other name reaches the engine's own methods unchanged. The engine pieces are
injected, so the routing is testable without the engine. The factory keeps the
original methods, so a second ``install_on`` is a no-op and ``uninstall`` restores them.
"""

from __future__ import annotations

import logging
from typing import Callable, Optional

from .backend_registry import MI355X_ATTN, V100_ALIAS

logger = logging.getLogger(__name__)

NAMES = (MI355X_ATTN, V100_ALIAS)
_SAVED = "_mi355x_attn_saved_methods"
_ROUTED = ("create_draft_extend_backend", "create_decode_backend")


class _Routes:
    """What the two rerouted methods do for our names."""

    def __init__(self, build: Callable, wrap: Callable, build_container: Optional[Callable]):
        self.build = build
        self.wrap = wrap
        self.build_container = build_container

    def create_draft_extend_backend(self, factory):
        runner = factory.draft_model_runner
        backend = self.build(runner)
        wrapped = None if backend is None else self.wrap(runner, backend)
        if wrapped is not None:
            for attr in ("prefill_attention_backend_str", "decode_attention_backend_str"):
                setattr(wrapped, attr, factory.draft_attn_backend)
        return wrapped

    def create_decode_backend(self, factory, engine_method):
        if int(factory.speculative_num_steps) < 2:
            # a one-step draft has no decode passes: whatever the engine returns for it
            return engine_method(factory)
        make = self.build_container
        if make is None:
            from .draft_decode import build_native as make
        return make(factory.draft_model_runner, int(factory.topk), int(factory.speculative_num_steps),
                    factory.draft_attn_backend)


def install_on(factory, build, wrap, build_container=None, names=NAMES) -> bool:
    """Reroute ``factory`` (the engine's DraftBackendFactory class) for ``names``; True if
    it was not rerouted before.

    ``build(runner)`` makes the backend, ``wrap(runner, backend)`` is the engine's
    draft-extend wrapper, ``build_container(runner, topk, steps, name)`` makes the
    multi-step decode container (default: ``draft_decode.build_native``).
    """
    if _SAVED in vars(factory):
        return False
    saved = {name: getattr(factory, name) for name in _ROUTED}
    routes = _Routes(build, wrap, build_container)
    ours = frozenset(names)

    def draft_extend(self):
        if self.draft_attn_backend in ours:
            return routes.create_draft_extend_backend(self)
        return saved["create_draft_extend_backend"](self)

    def decode(self):
        if self.draft_attn_backend in ours:
            return routes.create_decode_backend(self, saved["create_decode_backend"])
        return saved["create_decode_backend"](self)

    setattr(factory, _SAVED, saved)
    factory.create_draft_extend_backend = draft_extend
    factory.create_decode_backend = decode
    return True


def uninstall(factory) -> bool:
    """Give ``factory`` its own methods back; True if it was rerouted."""
    saved = vars(factory).get(_SAVED)
    if saved is None:
        return False
    for name, method in saved.items():
        setattr(factory, name, method)
    delattr(factory, _SAVED)
    return True


def install() -> bool:
    """Component hook: reroute the engine's draft factory when the engine is importable."""
    try:
        from sglang.srt.layers.attention.attention_registry import attn_backend_wrapper_for_draft_extend
        from sglang.srt.speculative import draft_utils
    except Exception as exc:  # noqa: BLE001 - report, never abort loading
        logger.info("attention_mi355x: draft backend hook skipped: %s", exc)
        return False
    from .backend_registry import build_backend

    changed = install_on(draft_utils.DraftBackendFactory, lambda runner: build_backend(MI355X_ATTN, runner),
                         attn_backend_wrapper_for_draft_extend)
    if changed:
        logger.info("attention_mi355x: a draft worker can now select %s", MI355X_ATTN)
    return changed
