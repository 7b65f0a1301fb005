"""Native multi-step draft decode on the split-KV kernel (the role of
sglang_restomod/attention/v100/draft_decode.py:46-208).

An EAGLE/NEXTN draft worker runs one attention pass per draft step; the engine's
multi-step container builds one flat ``kv_indptr`` / ``kv_indices`` pair per step
(row ``r`` owns ``kv_indices[kv_indptr[r]:kv_indptr[r+1]]``). The reference turns each
step's list into a page table for its page-granular kernel
(draft_decode_plan.py:42-78). The split-KV kernel here addresses tokens through a
table with a per-row start, so it reads the flat list itself: table ``kv_indices``
with row stride 1 and row starts ``kv_indptr[:-1]``, visible lengths
``diff(kv_indptr)``. No page table is built, and a step's metadata is two small
device ops (graph-safe when they target the fixed buffers of
``init_cuda_graph_state``).
"""

from __future__ import annotations

import logging
from typing import Optional

import torch

from . import draft_decode_plan as plan
from . import ops
from .backend import _EngineBase
from .backend_registry import env_flag

logger = logging.getLogger(__name__)

KV_DTYPES = (torch.float16, torch.bfloat16, torch.float8_e4m3fn, torch.float8_e5m2)
MODEL_DTYPES = (torch.float16, torch.bfloat16)


class MI355XDraftDecodeBackend(_EngineBase):
    """One draft step: the flat index list of the step plus the split-KV decode."""

    needs_cpu_seq_lens = False
    # the split-KV kernel balances on device; the attribute only sizes a buffer the
    # engine's container allocates for its own kernel
    max_kv_splits = 1

    def __init__(self, model_runner, topk: int, max_context_len: int, page_size: int, steps: int):
        if _EngineBase is not object:
            super().__init__()
        self.topk = int(topk)
        self.device = torch.device(model_runner.device)
        self.token_to_kv_pool = model_runner.token_to_kv_pool
        self.page_size = int(page_size)
        self.max_context_len = int(max_context_len)
        self.steps = int(steps)
        self.native_kv_write = env_flag("SGLANG_MI355X_NATIVE_KV_WRITE", "0")
        self._table: Optional[torch.Tensor] = None
        self._row_index: Optional[torch.Tensor] = None
        self._seq_lens: Optional[torch.Tensor] = None
        self._rows_used = 0
        # the split-KV workspace grows with the head dim: sized for the model's (the
        # largest supported one when the runner does not say), grown for a wider layer
        model_config = getattr(model_runner, "model_config", None)
        self.head_dim = int(getattr(model_config, "head_dim", max(plan.SUPPORTED_HEAD_DIMS)))
        self._workspace: Optional[torch.Tensor] = None
        self._workspace_dim = 0
        self._graph_rows = 0

    # ---- metadata ----
    def refresh(self, kv_indptr: torch.Tensor, kv_indices: torch.Tensor) -> int:
        """Point this step at its flat index list; returns the rows it serves."""
        if kv_indices.dtype != torch.int32:
            raise ValueError("kv_indices must be int32")
        rows = max(int(kv_indptr.numel()) - 1, 0)
        starts = kv_indptr[:rows]
        lens = kv_indptr[1:rows + 1] - starts
        if self._graph_rows:
            # fixed buffers, so that a captured decode reads this step's rows at replay
            if rows > self._graph_rows:
                raise ValueError(f"{rows} draft rows exceed the graph capacity {self._graph_rows}")
            self._g_row_index[:rows].copy_(starts)
            self._g_seq_lens[:rows].copy_(lens)
            self._row_index, self._seq_lens = self._g_row_index[:rows], self._g_seq_lens[:rows]
        else:
            self._row_index, self._seq_lens = starts.to(torch.int64), lens.to(torch.int32)
        base = kv_indices if kv_indices.numel() else torch.zeros(1, dtype=torch.int32, device=kv_indptr.device)
        # token table with row stride 1: position p of row r is kv_indices[kv_indptr[r] + p]
        self._table = torch.as_strided(base, (base.numel(), 1), (1, 1))
        self._rows_used = rows
        return rows

    def init_forward_metadata(self, forward_batch) -> None:
        spec_info = forward_batch.spec_info
        if spec_info is None or getattr(spec_info, "kv_indptr", None) is None:
            return
        self.refresh(spec_info.kv_indptr, spec_info.kv_indices)

    def init_forward_metadata_out_graph(self, forward_batch, in_capture: bool = False) -> None:
        self.init_forward_metadata(forward_batch)

    def init_cuda_graph_state(self, max_bs: int, max_num_tokens: int, kv_indices_buf=None,
                              cuda_graph_num_kv_splits_buf=None) -> None:
        rows = max(int(max_bs) * self.topk, 1)
        self._g_row_index = torch.zeros(rows, dtype=torch.int64, device=self.device)
        self._g_seq_lens = torch.zeros(rows, dtype=torch.int32, device=self.device)
        self._graph_rows = rows
        if self.device.type == "cuda":
            self._workspace = ops.splitkv_workspace(self.device, head_dim=self.head_dim)
            self._workspace_dim = self.head_dim

    def get_cuda_graph_seq_len_fill_value(self) -> int:
        return 1

    # ---- forward ----
    def forward_decode(self, q, k, v, layer, forward_batch, save_kv_cache: bool = True, **kwargs):
        rows = q.shape[0]
        if rows != self._rows_used:
            raise RuntimeError("draft decode metadata does not match the query rows: "
                               f"{self._rows_used} rows planned, {rows} seen")
        if kwargs.get("sinks") is not None:
            raise NotImplementedError("draft decode does not carry attention sinks")
        reason = plan.layer_shape_reason(layer)
        if reason is not None:
            raise NotImplementedError(f"draft decode cannot serve layer {layer.layer_id}: {reason}")
        if save_kv_cache and k is not None:
            if self.native_kv_write:
                k_cache, v_cache = self.token_to_kv_pool.get_kv_buffer(layer.layer_id)
                ks = float(layer.k_scale_float) if getattr(layer, "k_scale", None) is not None else None
                vs = float(layer.v_scale_float) if getattr(layer, "v_scale", None) is not None else None
                hkv, d = int(layer.tp_k_head_num), int(layer.head_dim)
                ops.set_kv_buffer(k_cache, v_cache, forward_batch.out_cache_loc,
                                  k.reshape(-1, hkv, d), v.reshape(-1, hkv, d), ks, vs)
            else:
                self.token_to_kv_pool.set_kv_buffer(layer, forward_batch.out_cache_loc, k, v,
                                                    layer.k_scale, layer.v_scale)
        hq, d = int(layer.tp_q_head_num), int(layer.qk_head_dim)
        k_cache, v_cache = self.token_to_kv_pool.get_kv_buffer(layer.layer_id)
        out_dtype = q.dtype
        q3 = q.reshape(rows, hq, d)
        if k_cache.dtype not in (torch.float8_e4m3fn, torch.float8_e5m2) and k_cache.dtype != q3.dtype:
            q3 = q3.to(k_cache.dtype)
        out = torch.empty(q3.shape, dtype=q3.dtype, device=q3.device)
        if rows:
            ks = float(layer.k_scale_float) if getattr(layer, "k_scale", None) is not None else 1.0
            vs = float(layer.v_scale_float) if getattr(layer, "v_scale", None) is not None else 1.0
            if q3.is_cuda and (self._workspace is None or self._workspace_dim < d):
                self._workspace = ops.splitkv_workspace(q3.device, head_dim=d)
                self._workspace_dim = d
            ops.grouped_decode_forward(
                q3, k_cache, v_cache, self._table, self._seq_lens, softmax_scale=float(layer.scaling),
                k_scale=ks, v_scale=vs, out=out, row_index=self._row_index, page_size=1,
                workspace=self._workspace)
        out = out.reshape(rows, hq * d)
        return out if out.dtype == out_dtype else out.to(out_dtype)

    def forward(self, q, k, v, layer, forward_batch, save_kv_cache: bool = True, **kwargs):
        return self.forward_decode(q, k, v, layer, forward_batch, save_kv_cache=save_kv_cache, **kwargs)


def make_multi_step_backend(base_cls):
    """The engine's per-step draft container (``base_cls``, the engine's
    TritonMultiStepDraftBackend) with split-KV children: its index builder and graph
    state stay the engine's, only the attention children change
    (draft_decode.py:172-208 of the reference)."""

    class MI355XMultiStepDraftBackend(base_cls):
        def __init__(self, model_runner, topk, speculative_num_steps, stamp):
            super().__init__(model_runner, topk, speculative_num_steps)
            self.attn_backends = [
                MI355XDraftDecodeBackend(model_runner, topk, self.max_context_len, model_runner.page_size,
                                         speculative_num_steps)
                for _ in range(self.speculative_num_steps - 1)
            ]
            self.prefill_attention_backend_str = stamp
            self.decode_attention_backend_str = stamp
            for child in self.attn_backends:
                child.prefill_attention_backend_str = stamp
                child.decode_attention_backend_str = stamp

        def init_forward_metadata_out_graph(self, forward_batch, in_capture: bool = False):
            # capture plans through the engine's builder; replay refills its index
            # buffers, then each child re-points at its step's list
            if in_capture:
                return super().init_forward_metadata_out_graph(forward_batch, in_capture=True)

            def call_fn(step, batch):
                self.attn_backends[step].init_forward_metadata(batch)

            self.common_template(forward_batch, None, call_fn)

    return MI355XMultiStepDraftBackend


def unsupported_reason(model_runner, topk: int, env=None, draft_window=(0, 0), layers=None) -> Optional[str]:
    """Why the split-KV draft path cannot serve this launch, or None
    (reference: draft_decode.py:216-251)."""
    if not plan.native_enabled(env):
        return f"disabled_by_env({plan.ENV_FLAG})"
    if int(getattr(model_runner, "page_size", 1)) != plan.PAGE_SIZE:
        return f"page_size({model_runner.page_size})"
    if getattr(model_runner, "kv_cache_dtype", None) not in KV_DTYPES:
        return f"kv_dtype({getattr(model_runner, 'kv_cache_dtype', None)})"
    model_dtype = getattr(getattr(model_runner, "model_config", None), "dtype", None)
    if model_dtype is not None and model_dtype not in MODEL_DTYPES:
        return f"model_dtype({model_dtype})"
    window, sink = draft_window
    if window or sink:
        return f"draft_window(window={window},sink={sink})"
    native_window = getattr(model_runner, "sliding_window_size", None)
    if native_window is not None and native_window > 0:
        return f"draft_sliding_window({native_window})"
    translator = getattr(model_runner, "kv_index_translator", None)
    if getattr(translator, "is_translating", False):
        return "kv_index_translation"
    if getattr(model_runner.token_to_kv_pool, "full_to_swa_index_mapping", None) is not None:
        return "swa_kv_pool"
    if layers is None:
        layers = [m for m in model_runner.model.modules() if hasattr(m, "tp_q_head_num") and hasattr(m, "layer_id")]
    if not layers:
        return "no_attention_layers"
    for layer in layers:
        reason = plan.layer_shape_reason(layer)
        if reason is not None:
            return f"layer{layer.layer_id}:{reason}"
    return None


def build_native(model_runner, topk: int, speculative_num_steps: int, stamp: str, base_cls=None):
    """The split-KV draft container, or None to keep the engine's own."""
    window = (0, 0)
    if base_cls is None:
        from sglang.srt.layers.attention.triton_backend import TritonMultiStepDraftBackend as base_cls
        from sglang.srt.speculative.spec_utils import resolve_draft_decode_window

        window = resolve_draft_decode_window(model_runner)
    reason = unsupported_reason(model_runner, topk, draft_window=window)
    if reason is not None:
        logger.info("attention_mi355x: draft decode stays on the engine's backend (%s)", reason)
        return None
    logger.info("attention_mi355x: draft decode on the split-KV kernel")
    return make_multi_step_backend(base_cls)(model_runner, topk, speculative_num_steps, stamp)
