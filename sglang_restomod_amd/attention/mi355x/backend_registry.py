"""Register the backend with the engine (contract of
sglang_restomod/attention/v100/backend_registry.py:104-162).

The engine publishes two hooks: ``register_attention_backend(name)(factory)``
fills ``ATTENTION_BACKENDS`` and ``add_attention_backend_choices`` extends the
list behind ``--attention-backend``. ``install`` takes them as keywords so tests
inject fakes; with none given it imports them from sglang. It is idempotent:
a second call changes nothing and returns False. The factory imports the
backend lazily, so registering never pulls in torch or the HIP library.
"""

from __future__ import annotations

import logging
import os
from collections.abc import Callable, Iterable, Mapping, MutableSequence

logger = logging.getLogger(__name__)

MI355X_ATTN = "mi355x_attn"
V100_ALIAS = "tilelang_fa_v100"
ENV_ALIAS = "SGLANG_MI355X_ATTN_ALIAS_V100"


def env_flag(name: str, default: str, env: Mapping[str, str] | None = None) -> bool:
    """Strict boolean env flag: 0/false/off/no or 1/true/on/yes, anything else raises."""
    raw = (os.environ if env is None else env).get(name, default)
    value = raw.strip().lower()
    if value in ("1", "true", "on", "yes"):
        return True
    if value in ("0", "false", "off", "no"):
        return False
    raise ValueError(f"{name} must be a boolean value, got {value!r}.")


def _make_backend(runner, skip_prefill: bool = False):
    from .backend import MI355XAttnBackend

    return MI355XAttnBackend(runner, skip_prefill=skip_prefill)


def backend_names(env: Mapping[str, str] | None = None) -> tuple[str, ...]:
    names = (MI355X_ATTN,)
    if env_flag(ENV_ALIAS, "0", env):
        names += (V100_ALIAS,)
    return names


def build_backend(name: str, runner):
    """Construct a registered backend by name (for draft factories that keep their own map)."""
    if name not in (MI355X_ATTN, V100_ALIAS):
        raise KeyError(name)
    return _make_backend(runner)


def _engine_hooks():
    from sglang.srt.arg_groups import choices
    from sglang.srt.layers.attention import attention_registry

    return (
        attention_registry.ATTENTION_BACKENDS,
        attention_registry.register_attention_backend,
        choices.ATTENTION_BACKEND_CHOICES,
        choices.add_attention_backend_choices,
    )


def install(
    *,
    registry: MutableSequence[str] | Mapping[str, Callable] | None = None,
    register: Callable[[str], Callable] | None = None,
    choices: Iterable[str] | None = None,
    extend_choices: Callable[[Iterable[str]], None] | None = None,
    env: Mapping[str, str] | None = None,
) -> bool:
    """Register the backend name(s); True if anything changed."""
    if registry is None or register is None or choices is None or extend_choices is None:
        hooks = _engine_hooks()
        registry = hooks[0] if registry is None else registry
        register = hooks[1] if register is None else register
        choices = hooks[2] if choices is None else choices
        extend_choices = hooks[3] if extend_choices is None else extend_choices
    changed = False
    missing = []
    for name in backend_names(env):
        if name not in registry:
            register(name)(_make_backend)
            changed = True
        if name not in choices:
            missing.append(name)
    if missing:
        extend_choices(missing)
        changed = True
    if changed:
        logger.info("attention_mi355x: registered backend(s) %s", ", ".join(backend_names(env)))
    return changed


def install_draft_choices() -> bool:
    """Let ``--speculative-draft-attention-backend`` name this backend (engine hook, if present)."""
    try:
        from sglang.srt.arg_groups.choices import add_draft_attention_backend_choices
    except Exception as exc:  # noqa: BLE001 - never abort loading
        logger.info("attention_mi355x: draft backend choices skipped: %s", exc)
        return False
    add_draft_attention_backend_choices([MI355X_ATTN])
    return True
