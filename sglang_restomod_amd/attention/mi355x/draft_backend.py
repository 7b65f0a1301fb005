"""Let a draft worker name this backend (the contract of
sglang_restomod/attention/v100/draft_backend.py:31-83).

The engine builds a draft worker's attention backends from a fixed name map in its
``DraftBackendFactory``. ``install_on`` patches the factory so that
``--speculative-draft-attention-backend mi355x_attn`` resolves:

* draft **extend** gets ``MI355XAttnBackend`` (wrapped by the engine's draft-extend
  wrapper): a few rows per request over the whole prefix, which the backend serves
  with the split-KV verify kernel;
* draft **decode** (more than one speculative step) gets the split-KV multi-step
  container of ``draft_decode``, or the engine's Triton container when
  ``draft_decode.unsupported_reason`` names a reason.

The hooks are injected so the patch is testable without the engine; patching twice
changes nothing.
"""

from __future__ import annotations

import logging

from .backend_registry import MI355X_ATTN, V100_ALIAS

logger = logging.getLogger(__name__)

FLAG = "_restomod_mi355x_draft"
DRAFT_DECODE_FALLBACK = "triton"
NAMES = (MI355X_ATTN, V100_ALIAS)


def install_on(factory, build, wrap, build_native=None, names=NAMES) -> bool:
    """Patch ``factory`` (the engine's DraftBackendFactory class); True if anything changed.

    ``build(runner)`` returns the backend, ``wrap(runner, backend)`` is the engine's
    draft-extend wrapper, ``build_native(runner, topk, steps, stamp)`` returns the
    split-KV draft-decode container or None.
    """
    if getattr(factory, FLAG, False):
        return False
    original_extend = factory.create_draft_extend_backend
    original_decode = factory.create_decode_backend

    def create_draft_extend_backend(self):
        if self.draft_attn_backend not in names:
            return original_extend(self)
        backend = build(self.draft_model_runner)
        if backend is None:
            return None
        wrapped = wrap(self.draft_model_runner, backend)
        if wrapped is not None:
            wrapped.prefill_attention_backend_str = self.draft_attn_backend
            wrapped.decode_attention_backend_str = self.draft_attn_backend
        return wrapped

    def create_decode_backend(self):
        if self.draft_attn_backend not in names:
            return original_decode(self)
        if self.speculative_num_steps > 1:
            builder = build_native
            if builder is None:
                from .draft_decode import build_native as builder
            native = builder(self.draft_model_runner, self.topk, self.speculative_num_steps, self.draft_attn_backend)
            if native is not None:
                return native
        saved = self.draft_attn_backend
        self.draft_attn_backend = DRAFT_DECODE_FALLBACK
        try:
            return original_decode(self)
        finally:
            self.draft_attn_backend = saved

    factory.create_draft_extend_backend = create_draft_extend_backend
    factory.create_decode_backend = create_decode_backend
    setattr(factory, FLAG, True)
    return True


def install() -> bool:
    """Component hook: patch the engine's draft factory when the engine is importable."""
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
