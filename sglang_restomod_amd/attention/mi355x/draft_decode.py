"""Multi-step speculative draft decode on the split-KV kernel.

Role: the draft worker's multi-step attention container (the reference's
NativeMultiStepDraftBackend, sglang_restomod/attention/v100/draft_decode.py:46-208, which
keeps the engine's own container for its per-step index lists and converts every
step's list into a page table, draft_decode_plan.py:42-78).

An EAGLE/NEXTN draft worker runs ``steps - 1`` attention passes per draft round. Pass
``i`` of branch ``k`` of request ``b`` attends over the request's prefix (its
``seq_lens[b]`` cached tokens) and the first ``i + 1`` draft tokens of the branch. The
engine stores the draft tokens in ``req_to_token`` right after the prefix: branch
``k``'s ``steps`` tokens start at position ``seq_lens[b] + k * steps``.

So every pass reads the same key rows, only more of each row:

* top-k 1 over a full-attention pool: the rows *are* the requests' ``req_to_token``
  rows; pass ``i`` reads ``seq_lens[b] + i + 1`` entries. Nothing is built.
* otherwise (several branches, or an SWA pool whose slots need translating): one
  ``ma_draft_table`` launch per round writes ``[bs * topk, width]`` rows, prefix then
  branch tokens, and every pass shares them.

Per round that is at most one small gather instead of a flat index list per step.
Every quantity lives on the device, so rounds replay from a captured graph once
``init_cuda_graph_state`` has fixed the buffers.

Served natively: any page size with top-k 1 (``req_to_token`` is token-granular, and
a single branch's tokens follow the prefix), top-k > 1 at page size 1, fp16 / bf16 /
e4m3fn / e5m2 pools, SWA pools, and sliding-window draft layers (the layer's window,
the kernel's visible-key rule). Anything else raises ``NotImplementedError`` at
construction: there is no fall-back to another backend.
"""

from __future__ import annotations

import logging
from dataclasses import dataclass
from typing import Optional

import torch

from . import draft_decode_plan as plan
from . import ops
from .backend import FP8_KV, _EngineBase, _is_encoder_only
from .backend_registry import env_flag
from .masks import resolve_layer_mask

logger = logging.getLogger(__name__)

KV_DTYPES = (torch.float16, torch.bfloat16) + FP8_KV
MODEL_DTYPES = (torch.float16, torch.bfloat16)
ENV_NATIVE_KV_WRITE = "SGLANG_MI355X_NATIVE_KV_WRITE"


@dataclass
class DraftRows:
    """Key rows of one draft round (or of one pass given as a flat index list).

    Pass ``i`` of row ``r`` reads ``table[row_index[r] if row_index is not None else r,
    : lens[i, r]]``. ``swa_table`` holds the same rows translated into an SWA pool's
    slots (row ``r``), for sliding-window layers of a hybrid pool.
    """

    table: torch.Tensor
    row_index: Optional[torch.Tensor]
    lens: torch.Tensor  # [passes, rows] int32
    swa_table: Optional[torch.Tensor] = None
    swa_row_index: Optional[torch.Tensor] = None  # row of swa_table per query row (None: row r)
    max_len: int = 0  # the longest row when the host knows it (eager rounds), else 0

    @property
    def rows(self) -> int:
        return int(self.lens.shape[1])

    @staticmethod
    def from_flat_lists(kv_indptr: torch.Tensor, kv_indices: torch.Tensor,
                        swa_mapping: Optional[torch.Tensor] = None) -> "DraftRows":
        """One pass whose rows come as a flat list (row ``r`` owns
        ``kv_indices[kv_indptr[r]:kv_indptr[r+1]]``): read in place as a table of row
        stride 1 with row starts ``kv_indptr[:-1]``. With an SWA pool's slot mapping
        (full-pool slot -> SWA slot), the list is also translated, on the device, for
        the pool's sliding-window layers."""
        if kv_indices.dtype != torch.int32:
            raise ValueError("kv_indices must be int32")
        rows = max(int(kv_indptr.numel()) - 1, 0)
        starts = kv_indptr[:rows].to(torch.int64)
        lens = (kv_indptr[1:rows + 1] - kv_indptr[:rows]).to(torch.int32).reshape(1, rows)
        base = kv_indices if kv_indices.numel() else torch.zeros(1, dtype=torch.int32, device=kv_indptr.device)
        table = torch.as_strided(base, (base.numel(), 1), (1, 1))
        swa_table = None
        if swa_mapping is not None:
            swa = swa_mapping[base.to(torch.int64)].to(torch.int32)
            swa_table = torch.as_strided(swa, (swa.numel(), 1), (1, 1))
        return DraftRows(table=table, row_index=starts, lens=lens, swa_table=swa_table,
                         swa_row_index=starts if swa_table is not None else None)


def support_gaps(model_runner, topk: int, draft_window=(0, 0), layers=None) -> list[str]:
    """Every reason the split-KV draft path cannot serve this draft worker (empty: it can)."""
    gaps = []
    kv_dtype = getattr(model_runner, "kv_cache_dtype", None)
    if kv_dtype not in KV_DTYPES:
        gaps.append(f"KV cache dtype {kv_dtype} (served: fp16, bf16, e4m3fn, e5m2)")
    model_dtype = getattr(getattr(model_runner, "model_config", None), "dtype", None)
    if model_dtype is not None and model_dtype not in MODEL_DTYPES:
        gaps.append(f"model dtype {model_dtype} (served: fp16, bf16)")
    page_size = int(getattr(model_runner, "page_size", 1))
    if topk > 1 and page_size > 1:
        gaps.append(f"top-k {topk} at page size {page_size} (the engine's per-branch page layout "
                    "is served at page size 1 only)")
    window, sink = draft_window
    if window or sink:
        gaps.append(f"engine draft-decode window (window={window}, sink={sink}): its key selection "
                    "is the engine's and is not carried here")
    translator = getattr(model_runner, "kv_index_translator", None)
    if getattr(translator, "is_translating", False):
        gaps.append("KV index translation")
    for layer in layers or ():
        reason = plan.layer_shape_reason(layer)
        if reason is not None:
            gaps.append(f"layer {getattr(layer, 'layer_id', '?')}: {reason}")
    return gaps


class MI355XDraftDecodeBackend(_EngineBase):
    """Attention of one draft pass: the split-KV decode over its share of the round's rows."""

    needs_cpu_seq_lens = False
    # the engine sizes a split buffer for its own kernels from this attribute; the
    # split-KV kernel splits on the device
    max_kv_splits = 1

    def __init__(self, container: "MI355XMultiStepDraftBackend", step: int):
        if _EngineBase is not object:
            super().__init__()
        self.container = container
        self.step = int(step)
        self._own: Optional[DraftRows] = None  # rows handed to this pass alone (flat lists)

    # ---- metadata ----
    def rows(self) -> DraftRows:
        if self._own is not None:
            return self._own
        if self.container.current is None:
            raise RuntimeError("draft decode without metadata (init_forward_metadata first)")
        return self.container.current

    def use_flat_lists(self, kv_indptr: torch.Tensor, kv_indices: torch.Tensor) -> int:
        """Serve this pass from a flat index list instead of the round's rows; returns its rows."""
        self._own = DraftRows.from_flat_lists(kv_indptr, kv_indices, self.container.swa_mapping)
        return self._own.rows

    @staticmethod
    def table_for(rows: DraftRows, window: int):
        """(table, row_index) a layer reads: the SWA pool's translated rows for a
        sliding-window layer when the pool has them, else the full pool's rows."""
        if window >= 0 and rows.swa_table is not None:
            return rows.swa_table, rows.swa_row_index
        return rows.table, rows.row_index

    def init_forward_metadata(self, forward_batch) -> None:
        spec_info = getattr(forward_batch, "spec_info", None)
        if spec_info is not None and getattr(spec_info, "kv_indptr", None) is not None:
            self.use_flat_lists(spec_info.kv_indptr, spec_info.kv_indices)

    def init_forward_metadata_out_graph(self, forward_batch, in_capture: bool = False) -> None:
        self.init_forward_metadata(forward_batch)

    def get_cuda_graph_seq_len_fill_value(self) -> int:
        return 1

    # ---- forward ----
    def _save_kv(self, layer, loc, k, v) -> None:
        pool = self.container.token_to_kv_pool
        # an SWA pool translates the slots of its sliding-window layers in its own write
        if not self.container.native_kv_write or self.container.swa_mapping is not None:
            pool.set_kv_buffer(layer, loc, k, v, layer.k_scale, layer.v_scale)
            return
        k_cache, v_cache = pool.get_kv_buffer(layer.layer_id)
        ks = float(layer.k_scale_float) if getattr(layer, "k_scale", None) is not None else None
        vs = float(layer.v_scale_float) if getattr(layer, "v_scale", None) is not None else None
        hkv, d = int(layer.tp_k_head_num), int(layer.head_dim)
        ops.set_kv_buffer(k_cache, v_cache, loc, k.reshape(-1, hkv, d), v.reshape(-1, hkv, d), ks, vs)

    def forward_decode(self, q, k, v, layer, forward_batch, save_kv_cache: bool = True, **kwargs):
        if kwargs.get("sinks") is not None:
            raise NotImplementedError("draft decode does not carry attention sinks")
        reason = plan.layer_shape_reason(layer)
        if reason is not None:
            raise NotImplementedError(f"draft decode cannot serve layer {layer.layer_id}: {reason}")
        rows = self.rows()
        n = int(q.shape[0])
        if n != rows.rows:
            raise RuntimeError(f"draft decode metadata does not match the query rows: {rows.rows} planned, {n} seen")
        if save_kv_cache and k is not None:
            self._save_kv(layer, forward_batch.out_cache_loc, k, v)
        hq, d = int(layer.tp_q_head_num), int(layer.qk_head_dim)
        k_cache, v_cache = self.container.token_to_kv_pool.get_kv_buffer(layer.layer_id)
        q3 = q.reshape(n, hq, d)
        if k_cache.dtype not in FP8_KV and k_cache.dtype != q3.dtype:
            q3 = q3.to(k_cache.dtype)
        out = torch.empty(q3.shape, dtype=q3.dtype, device=q3.device)
        _, window = resolve_layer_mask(
            default_causal=True, is_cross_attention=bool(getattr(layer, "is_cross_attention", False)),
            is_encoder_only=_is_encoder_only(layer), sliding_window_size=getattr(layer, "sliding_window_size", None))
        if n:
            table, row_index = self.table_for(rows, window)
            ks = float(layer.k_scale_float) if getattr(layer, "k_scale", None) is not None else 1.0
            vs = float(layer.v_scale_float) if getattr(layer, "v_scale", None) is not None else 1.0
            ops.grouped_decode_forward(
                q3, k_cache, v_cache, table, rows.lens[0 if self._own is not None else self.step],
                softmax_scale=float(layer.scaling), k_scale=ks, v_scale=vs, out=out, row_index=row_index,
                page_size=1, sliding_window_size=window, max_seq_len_hint=rows.max_len,
                workspace=self.container.workspace(d))
        out = out.reshape(n, hq * d)
        return out if out.dtype == q.dtype else out.to(q.dtype)

    def forward(self, q, k, v, layer, forward_batch, save_kv_cache: bool = True, **kwargs):
        return self.forward_decode(q, k, v, layer, forward_batch, save_kv_cache=save_kv_cache, **kwargs)


class MI355XMultiStepDraftBackend:
    """The draft worker's multi-step container: ``attn_backends[i]`` serves draft pass ``i``.

    The engine calls ``init_forward_metadata`` (eager rounds),
    ``init_cuda_graph_state`` then ``init_forward_metadata_capture_cuda_graph`` /
    ``init_forward_metadata_replay_cuda_graph`` (graph rounds), or
    ``init_forward_metadata_out_graph``; each plans the round's rows once.
    """

    def __init__(self, model_runner, topk: int, speculative_num_steps: int, stamp: str = "mi355x_attn",
                 draft_window=(0, 0), layers=None):
        self.topk = int(topk)
        self.speculative_num_steps = int(speculative_num_steps)
        if self.topk < 1 or self.speculative_num_steps < 2:
            raise ValueError("a multi-step draft needs topk >= 1 and at least two steps")
        if layers is None:
            model = getattr(model_runner, "model", None)
            layers = [m for m in model.modules() if hasattr(m, "tp_q_head_num")] if model is not None else []
        gaps = support_gaps(model_runner, self.topk, draft_window, layers)
        if gaps:
            raise NotImplementedError("mi355x_attn draft decode cannot serve this draft worker: " + "; ".join(gaps))
        self.device = torch.device(model_runner.device)
        self.req_to_token = model_runner.req_to_token_pool.req_to_token
        if self.req_to_token.dtype != torch.int32:
            raise ValueError("req_to_token must be int32")
        self.token_to_kv_pool = model_runner.token_to_kv_pool
        self.swa_mapping = getattr(self.token_to_kv_pool, "full_to_swa_index_mapping", None)
        self.native_kv_write = env_flag(ENV_NATIVE_KV_WRITE, "1")
        model_config = getattr(model_runner, "model_config", None)
        # the model's head dim sizes the workspace made before capture; without one, the
        # head dim with the largest split-KV workspace
        self.head_dim = int(getattr(model_config, "head_dim", max(ops.TUNED_HEAD_DIMS)))
        self.max_context_len = int(getattr(model_config, "context_len", self.req_to_token.shape[1]))
        self.passes = self.speculative_num_steps - 1
        self.attn_backends = [MI355XDraftDecodeBackend(self, i) for i in range(self.passes)]
        for obj in (self, *self.attn_backends):
            obj.prefill_attention_backend_str = stamp
            obj.decode_attention_backend_str = stamp
        self.current: Optional[DraftRows] = None
        self._ws: Optional[torch.Tensor] = None
        self._graph: Optional[dict] = None
        # eager rounds write their tables into these (grown as needed, reused every round:
        # the passes of one round run before the next round's table on the same stream)
        self._eager: dict = {}

    # ---- buffers ----
    def workspace(self, head_dim: int) -> torch.Tensor:
        """One split-KV workspace for every pass (the passes run one after another on the
        engine's stream), grown for a wider layer outside graph capture only."""
        need = ops.splitkv_workspace_bytes(self.device, head_dim)
        if self._ws is None or self._ws.numel() < need:
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError("the draft workspace must exist before graph capture (init_cuda_graph_state)")
            widest = max((head_dim, self.head_dim), key=lambda d: ops.splitkv_workspace_bytes(self.device, d))
            self._ws = ops.splitkv_workspace(self.device, head_dim=widest)
        return self._ws

    def _needs_table(self) -> bool:
        return self.topk > 1

    def _eager_buffer(self, name: str, rows: int, width: int) -> torch.Tensor:
        """A [rows, width] int32 view of the container's own buffer ``name`` for an eager
        round, grown (never shrunk) when a round needs more rows or a wider row."""
        buf = self._eager.get(name)
        if buf is None or buf.shape[0] < rows or buf.shape[1] < width:
            r = max(rows, buf.shape[0] if buf is not None else 0)
            w = max(width, buf.shape[1] if buf is not None else 0)
            buf = torch.empty(r, w, dtype=torch.int32, device=self.device)
            self._eager[name] = buf
        return buf[:rows, :width]

    def init_cuda_graph_state(self, max_bs: int, max_num_tokens: int = 0, kv_indices_buf=None,
                              cuda_graph_num_kv_splits_buf=None) -> None:
        rows = max(int(max_bs), 1) * self.topk
        width = int(self.req_to_token.shape[1])
        dev = self.device
        g = {
            "max_bs": max(int(max_bs), 1),
            "row_index": torch.zeros(max(int(max_bs), 1), dtype=torch.int64, device=dev),
            "lens": torch.zeros(self.passes, rows, dtype=torch.int32, device=dev),
            "table": torch.zeros(rows, width, dtype=torch.int32, device=dev) if self._needs_table() else None,
            "swa": torch.zeros(rows, width, dtype=torch.int32, device=dev) if self.swa_mapping is not None else None,
        }
        self._graph = g
        if dev.type == "cuda":
            self.workspace(self.head_dim)

    # ---- planning ----
    def plan(self, req_pool_indices: torch.Tensor, seq_lens: torch.Tensor, bs: Optional[int] = None,
             seq_lens_cpu=None, graph: bool = False) -> DraftRows:
        """The round's rows for ``bs`` requests (in graph buffers when ``graph``)."""
        bs = int(seq_lens.shape[0] if bs is None else bs)
        max_len = 0
        rows = bs * self.topk
        seq = seq_lens[:bs].to(torch.int32)
        req = req_pool_indices[:bs].to(torch.int64)
        per_row = seq.reshape(bs, 1).expand(bs, self.topk).reshape(rows)
        if graph:
            g = self._graph
            if g is None:
                raise RuntimeError("init_cuda_graph_state must run before graph capture")
            if bs > g["max_bs"]:
                raise ValueError(f"batch {bs} exceeds the graph capacity {g['max_bs']}")
            lens = g["lens"][:, :rows]
            g["row_index"][:bs].copy_(req)
            req = g["row_index"][:bs]
            width = int(self.req_to_token.shape[1])
        else:
            lens = torch.empty(self.passes, rows, dtype=torch.int32, device=seq.device)
            width = int(self.req_to_token.shape[1])
            if seq_lens_cpu is not None and len(seq_lens_cpu):
                width = min(width, int(max(int(s) for s in seq_lens_cpu[:bs])) + self.speculative_num_steps)
                max_len = width
        for i in range(self.passes):
            torch.add(per_row, i + 1, out=lens[i])
        table, row_index = self.req_to_token, req
        if self._needs_table():
            out = self._graph["table"][:rows] if graph else self._eager_buffer("table", rows, width)
            table = ops.draft_table(self.req_to_token, seq, self.topk, self.speculative_num_steps, row_index=req,
                                    out=out, width=width)
            row_index = None
        swa = None
        if self.swa_mapping is not None:
            out = self._graph["swa"][:rows] if graph else self._eager_buffer("swa", rows, width)
            swa = ops.draft_table(self.req_to_token, seq, self.topk, self.speculative_num_steps, row_index=req,
                                  mapping=self.swa_mapping, out=out, width=width)
        rows_md = DraftRows(table=table, row_index=row_index, lens=lens, swa_table=swa, max_len=max_len)
        self.current = rows_md
        for child in self.attn_backends:
            child._own = None
        return rows_md

    def init_forward_metadata(self, forward_batch) -> None:
        self.plan(forward_batch.req_pool_indices, forward_batch.seq_lens,
                  seq_lens_cpu=getattr(forward_batch, "seq_lens_cpu", None))

    def init_forward_metadata_capture_cuda_graph(self, forward_batch) -> None:
        self.plan(forward_batch.req_pool_indices, forward_batch.seq_lens, bs=forward_batch.batch_size, graph=True)

    def init_forward_metadata_replay_cuda_graph(self, forward_batch, bs: int) -> None:
        self.plan(forward_batch.req_pool_indices, forward_batch.seq_lens, bs=bs, graph=True)

    def init_forward_metadata_out_graph(self, forward_batch, in_capture: bool = False) -> None:
        if self._graph is None:
            self.init_forward_metadata(forward_batch)
        elif in_capture:
            self.init_forward_metadata_capture_cuda_graph(forward_batch)
        else:
            self.init_forward_metadata_replay_cuda_graph(forward_batch, forward_batch.batch_size)


def build_native(model_runner, topk: int, speculative_num_steps: int, stamp: str, draft_window=None,
                 layers=None) -> MI355XMultiStepDraftBackend:
    """The split-KV draft container for this draft worker (raises NotImplementedError
    naming every gap when it cannot serve it)."""
    if draft_window is None:
        draft_window = (0, 0)
        try:
            from sglang.srt.speculative.spec_utils import resolve_draft_decode_window
        except Exception:  # noqa: BLE001 - an engine without draft windows has none
            resolve_draft_decode_window = None
        if resolve_draft_decode_window is not None:
            draft_window = tuple(resolve_draft_decode_window(model_runner))
    container = MI355XMultiStepDraftBackend(model_runner, topk, speculative_num_steps, stamp,
                                            draft_window=draft_window, layers=layers)
    logger.info("attention_mi355x: draft decode of %d passes on the split-KV kernel (top-k %d)",
                container.passes, container.topk)
    return container
