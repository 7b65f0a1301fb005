"""MI355X attention backend: the engine-facing surface of the paged-attention path.

Mirrors the method surface of the V100 backend
(sglang_restomod/attention/v100/flash_attn_v100_backend.py:166-1307): metadata per
forward (``init_forward_metadata``, :567-621), graph-runner entry points
(``init_forward_metadata_out_graph`` :622-681, ``init_cuda_graph_state`` :684-729,
capture :731-782, replay :784-856), ``forward_decode`` (:1093-1115) and
``forward_extend`` (:1117-1304).

What differs by design:

* Every supported layer runs on the HIP kernels: decode, prefix-aware extend,
  linear target verify and draft extend. Nothing is delegated to another backend,
  and layers the kernels cannot serve (a head dim that is not a multiple of 16 up to
  512, logit soft-capping, attention sinks, cross-attention, tree-shaped verify) raise
  ``NotImplementedError`` naming the reason, instead of running elsewhere.
* The kernels address SGLang's ``req_to_token`` directly (page size 1,
  ``req_pool_indices`` as the row index), so the metadata is the engine's own
  tensors plus ``query_start_loc`` and the prefix lengths: no page table is built
  and nothing synchronises with the host (the reference reads
  ``seq_lens.max().item()`` here, :457). The extend kernel lists its row tiles on
  the device, and the sliding-window table of an SWA pool is translated on the
  device row by row (``ops.translate_slots``). Routing a draft extend to the verify
  kernel uses host-known shapes only (token and request counts), never device values.
* fp8 KV (e4m3fn / e5m2, per-tensor scale) is read directly by every kernel; the
  reference's fp16 prefill scratch (:277-330, gather at :1226-1253) is not needed.
"""

from __future__ import annotations

import logging
from dataclasses import dataclass
from typing import Optional

import torch

from . import ops
from .backend_registry import env_flag
from .draft_decode_plan import layer_shape_reason
from .masks import resolve_layer_mask

logger = logging.getLogger(__name__)

try:  # the engine's base class when the engine is installed
    from sglang.srt.layers.attention.base_attn_backend import AttentionBackend as _EngineBase
except Exception:  # noqa: BLE001 - standalone use and tests
    _EngineBase = object

FP8_KV = (torch.float8_e4m3fn, torch.float8_e5m2)
MODE_DECODE = "decode"
MODE_EXTEND = "extend"
MODE_VERIFY = "verify"
# new K/V go into the pool's buffers through this library's kernel (ops.set_kv_buffer: the
# same stored bytes as the pool's own set_kv_buffer); "0" calls the pool's method instead
ENV_NATIVE_KV_WRITE = "SGLANG_MI355X_NATIVE_KV_WRITE"


@dataclass
class MI355XForwardMetadata:
    """Per-forward metadata (the role of FlashAttnV100ExtendMetadata,
    flash_attn_v100_backend.py:144-163).

    ``table`` is ``req_to_token`` [rows, max_context] int32 and ``row_index`` the
    batch's ``req_pool_indices`` (int64), so position ``j`` of sequence ``b`` lives in
    pool slot ``table[row_index[b], j]``. ``swa_table`` / ``swa_row_index`` replace
    them for sliding-window layers whose KV lives in a separate SWA pool.
    """

    mode: str
    table: torch.Tensor
    row_index: torch.Tensor
    seq_lens: torch.Tensor
    query_start_loc: Optional[torch.Tensor] = None
    prefix_kv_lens: Optional[torch.Tensor] = None
    causal: bool = True
    max_q_per_seq: int = 1
    num_tokens: int = 0
    swa_table: Optional[torch.Tensor] = None
    swa_row_index: Optional[torch.Tensor] = None
    # the longest sequence when the host knows it (eager forwards), else 0: it only picks
    # the decode kernels, never the result
    max_seq_len: int = 0


def _mode_is(mode, name: str) -> bool:
    fn = getattr(mode, name, None)
    return bool(fn()) if callable(fn) else False


def _is_encoder_only(layer) -> bool:
    attn_type = getattr(layer, "attn_type", None)
    return getattr(attn_type, "name", str(attn_type)).upper().endswith("ENCODER_ONLY")


class MI355XAttnBackend(_EngineBase):
    """Paged GQA attention for MI355X over SGLang's token pool."""

    # decode metadata is built from device tensors only
    needs_cpu_seq_lens: bool = False

    def __init__(self, model_runner, skip_prefill: bool = False):
        if _EngineBase is not object:
            super().__init__()
        self.model_runner = model_runner
        self.device = torch.device(model_runner.device)
        self.page_size = int(model_runner.page_size)
        self.max_context_len = int(model_runner.model_config.context_len)
        self.req_to_token_pool = model_runner.req_to_token_pool
        self.req_to_token = model_runner.req_to_token_pool.req_to_token
        self.token_to_kv_pool = model_runner.token_to_kv_pool
        self.skip_prefill = skip_prefill
        self.kv_cache_dtype = getattr(model_runner, "kv_cache_dtype", None)
        head_dim = int(model_runner.model_config.head_dim)
        v_head_dim = int(getattr(model_runner.model_config, "v_head_dim", head_dim))
        if head_dim != v_head_dim or not ops.head_dim_supported(head_dim):
            raise NotImplementedError(
                f"mi355x_attn serves a head_dim that is a multiple of {ops.HEAD_DIM_MULTIPLE} up to "
                f"{ops.MAX_HEAD_DIM} with equal q/k and v dims (model has qk {head_dim}, v {v_head_dim})")
        if self.req_to_token.dtype != torch.int32:
            raise ValueError("req_to_token must be int32")
        self.head_dim = head_dim
        self.native_kv_write = env_flag(ENV_NATIVE_KV_WRITE, "1")
        self.forward_metadata: Optional[MI355XForwardMetadata] = None
        self._workspace: Optional[torch.Tensor] = None
        self._extend_ws: Optional[torch.Tensor] = None
        # graph buffers (init_cuda_graph_state)
        self._cg_max_bs = 0
        self._cg_row_index: Optional[torch.Tensor] = None
        self._cg_seq_lens: Optional[torch.Tensor] = None
        self._cg_query_start_loc: Optional[torch.Tensor] = None
        self._cg_prefix_kv_lens: Optional[torch.Tensor] = None
        self._cg_swa_table: Optional[torch.Tensor] = None
        self._cg_rows_per_req = 0  # rows per request of the captured draft-extend graphs

    # ------------------------------------------------------------------
    # Mode routing (reference: _uses_native_linear_verify :332-380,
    # _uses_native_draft_extend :382-416)
    # ------------------------------------------------------------------
    def _spec_topk(self) -> int:
        server_args = getattr(self.model_runner, "server_args", None)
        topk = getattr(server_args, "speculative_eagle_topk", None)
        return 1 if topk is None else int(topk)

    def _check_linear_verify(self) -> None:
        """Target verify is served as a linear chain; a token tree needs a custom mask."""
        spec = getattr(self.model_runner, "spec_algorithm", None)
        dflash = _mode_is(spec, "is_dflash_family")
        if not dflash and self._spec_topk() > 1:
            raise NotImplementedError(
                "mi355x_attn serves linear speculative verification only "
                f"(speculative_eagle_topk={self._spec_topk()} builds a token tree)")

    def _has_swa_pool(self) -> bool:
        pool = self.token_to_kv_pool
        return (hasattr(pool, "translate_loc_from_full_to_swa")
                and getattr(pool, "full_to_swa_index_mapping", None) is not None)

    # ------------------------------------------------------------------
    # Metadata (reference: _build_extend_metadata :432-565, init_forward_metadata :567-621)
    # ------------------------------------------------------------------
    def _swa_rows(self, row_index: torch.Tensor, seq_lens: torch.Tensor,
                  out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """req_to_token rows translated to SWA-pool slots on the device, [B, width] int32,
        each row up to its own length (reference :460-503 gathers up to the longest
        sequence, read with .item())."""
        width = int(self.req_to_token.shape[1]) if out is None else min(int(out.shape[1]),
                                                                        int(self.req_to_token.shape[1]))
        return ops.translate_slots(self.req_to_token, seq_lens, self.token_to_kv_pool.full_to_swa_index_mapping,
                                   row_index=row_index, out=out, width=width)

    def build_metadata(
        self,
        mode: str,
        req_pool_indices: torch.Tensor,
        seq_lens: torch.Tensor,
        extend_seq_lens: Optional[torch.Tensor] = None,
        extend_prefix_lens: Optional[torch.Tensor] = None,
        max_q_per_seq: Optional[int] = None,
        seq_lens_cpu=None,
    ) -> MI355XForwardMetadata:
        row_index = req_pool_indices.to(torch.int64)
        seq = seq_lens.to(torch.int32)
        md = MI355XForwardMetadata(mode=mode, table=self.req_to_token, row_index=row_index, seq_lens=seq)
        if seq_lens_cpu is not None and len(seq_lens_cpu):
            md.max_seq_len = max(0, int(max(int(x) for x in seq_lens_cpu)))
        if mode != MODE_DECODE:
            ext = extend_seq_lens.to(torch.int32)
            pre = extend_prefix_lens.to(torch.int32)
            # a warm-up batch may carry a decode fill value in seq_lens; prefix + extend
            # is the length the kernels must see (reference :452-455)
            md.seq_lens = torch.maximum(seq, pre + ext)
            md.prefix_kv_lens = pre
            qsl = torch.zeros(seq.shape[0] + 1, dtype=torch.int32, device=seq.device)
            torch.cumsum(ext, dim=0, dtype=torch.int32, out=qsl[1:])
            md.query_start_loc = qsl
            # the extend kernel lists its row tiles on the device; only the verifier's
            # grid needs the longest chain, which callers pass (0: not known)
            md.max_q_per_seq = int(max_q_per_seq) if max_q_per_seq is not None else 0
        if self._has_swa_pool():
            md.swa_table = self._swa_rows(row_index, md.seq_lens)
            md.swa_row_index = torch.arange(row_index.shape[0], dtype=torch.int64, device=row_index.device)
        return md

    def init_forward_metadata(self, forward_batch) -> None:
        mode = forward_batch.forward_mode
        seq_lens_cpu = getattr(forward_batch, "seq_lens_cpu", None)
        if _mode_is(mode, "is_decode_or_idle"):
            self.forward_metadata = self.build_metadata(
                MODE_DECODE, forward_batch.req_pool_indices, forward_batch.seq_lens,
                seq_lens_cpu=seq_lens_cpu)
            return
        if _mode_is(mode, "is_target_verify"):
            self._check_linear_verify()
            n = int(forward_batch.spec_info.draft_token_num)
            prefix = forward_batch.seq_lens
            ext = torch.full_like(prefix, n)
            cpu = None if seq_lens_cpu is None else [int(s) + n for s in seq_lens_cpu]
            self.forward_metadata = self.build_metadata(
                MODE_VERIFY, forward_batch.req_pool_indices, prefix + n, ext, prefix,
                max_q_per_seq=n, seq_lens_cpu=cpu)
            return
        ext_cpu = getattr(forward_batch, "extend_seq_lens_cpu", None)
        max_q = int(max(ext_cpu)) if ext_cpu is not None and len(ext_cpu) else None
        md = self.build_metadata(
            MODE_EXTEND, forward_batch.req_pool_indices, forward_batch.seq_lens,
            forward_batch.extend_seq_lens, forward_batch.extend_prefix_lens,
            max_q_per_seq=max_q, seq_lens_cpu=seq_lens_cpu)
        # a draft extend is a few rows per request over the whole prefix, the verify kernel's
        # shape. Routed by host-known sizes (the reference reads the longest chain with
        # .item() instead, _paged_adapter.py:613-617): at most VERIFY_MAX_Q_PER_SEQ rows per
        # request on average; the longest chain, when the host has it, picks the row groups.
        draft = _mode_is(mode, "is_draft_extend_v2") or _mode_is(mode, "is_draft_extend")
        batch = int(forward_batch.req_pool_indices.shape[0])
        tokens = int(forward_batch.out_cache_loc.shape[0])
        if draft and batch and tokens <= batch * ops.VERIFY_MAX_Q_PER_SEQ:
            md.mode = MODE_VERIFY
            md.max_q_per_seq = max(1, min(max_q if max_q else tokens, ops.VERIFY_MAX_Q_PER_SEQ))
        self.forward_metadata = md

    # ------------------------------------------------------------------
    # Graph capture / replay (reference :622-856)
    # ------------------------------------------------------------------
    def get_cuda_graph_seq_len_fill_value(self) -> int:
        return 1

    def get_verify_buffers_to_fill_after_draft(self):
        # a linear chain needs no custom mask
        return [None, None]

    def update_verify_buffers_to_fill_after_draft(self, spec_info, cuda_graph_bs: Optional[int]):
        return None

    def splitkv_workspace(self) -> torch.Tensor:
        if self.device.type != "cuda":
            raise ValueError("the MI355X attention operators need device tensors "
                             f"(backend device is {self.device})")
        if self._workspace is None:
            self._workspace = ops.splitkv_workspace(self.device, head_dim=self.head_dim)
        return self._workspace

    def _workspace_for(self, mode: str, num_tokens: int, hq: int, hkv: int, batch: int) -> torch.Tensor:
        """The split-KV workspace, which also holds an extend call's work list (8 bytes
        per row tile); a larger buffer only for a batch whose list does not fit."""
        ws = self.splitkv_workspace()
        if mode == MODE_VERIFY:
            return ws
        need = ops.extend_workspace_bytes(num_tokens, hq, hkv, batch)
        if ws.numel() >= need:
            return ws
        if self._extend_ws is None or self._extend_ws.numel() < need:
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError(f"an extend of {num_tokens} tokens needs {need} workspace bytes; "
                                   "capture smaller batches")
            self._extend_ws = ops.extend_workspace(self.device, num_tokens, hq, hkv, batch)
        return self._extend_ws

    def init_cuda_graph_state(self, max_bs: int, max_num_tokens: int, kv_indices_buf=None) -> None:
        dev = self.device
        self._cg_max_bs = int(max_bs)
        self._cg_row_index = torch.zeros(max_bs, dtype=torch.int64, device=dev)
        self._cg_seq_lens = torch.zeros(max_bs, dtype=torch.int32, device=dev)
        self._cg_query_start_loc = torch.zeros(max_bs + 1, dtype=torch.int32, device=dev)
        self._cg_prefix_kv_lens = torch.zeros(max_bs, dtype=torch.int32, device=dev)
        if self._has_swa_pool():
            self._cg_swa_table = torch.zeros(max_bs, self.max_context_len, dtype=torch.int32, device=dev)
        if dev.type == "cuda":
            self.splitkv_workspace()  # allocated before any capture

    def _fill_graph_metadata(self, bs: int, num_tokens: int, req_pool_indices, seq_lens,
                             forward_mode, spec_info) -> None:
        if self._cg_seq_lens is None:
            raise RuntimeError("init_cuda_graph_state must run before graph capture")
        if bs > self._cg_max_bs:
            raise ValueError(f"batch {bs} exceeds the graph capacity {self._cg_max_bs}")
        self._cg_row_index[:bs].copy_(req_pool_indices[:bs])
        seq = seq_lens[:bs].to(torch.int32)
        if _mode_is(forward_mode, "is_decode_or_idle"):
            self._cg_seq_lens[:bs].copy_(seq)
            mode, max_q = MODE_DECODE, 1
        elif _mode_is(forward_mode, "is_target_verify"):
            self._check_linear_verify()
            n = int(spec_info.draft_token_num)
            self._cg_prefix_kv_lens[:bs].copy_(seq)
            self._cg_seq_lens[:bs].copy_(seq + n)
            self._cg_query_start_loc[: bs + 1].copy_(
                torch.arange(0, (bs + 1) * n, n, dtype=torch.int32, device=seq.device))
            mode, max_q = MODE_VERIFY, n
        elif _mode_is(forward_mode, "is_draft_extend_v2") or _mode_is(forward_mode, "is_draft_extend"):
            # a captured draft extend runs a fixed number of rows per request (the graph's
            # num_tokens / bs, the layout graph runners pad to): request b's rows are the
            # last n positions of its seq_lens[b] keys. Built on the device in the fixed
            # buffers, so a replay only refreshes them. (The reference hands these graphs to
            # another backend, :747, :801.)
            if bs <= 0 or num_tokens % bs:
                raise NotImplementedError(
                    f"a captured draft extend needs the same number of rows per request ({num_tokens} tokens "
                    f"over {bs} requests)")
            n = int(num_tokens) // bs
            self._cg_rows_per_req = n
            self._cg_seq_lens[:bs].copy_(seq)
            torch.sub(seq, n, out=self._cg_prefix_kv_lens[:bs])
            self._cg_prefix_kv_lens[:bs].clamp_(min=0)
            self._cg_query_start_loc[: bs + 1].copy_(
                torch.arange(0, (bs + 1) * n, n, dtype=torch.int32, device=seq.device))
            mode, max_q = (MODE_VERIFY, n) if n <= ops.VERIFY_MAX_Q_PER_SEQ else (MODE_EXTEND, n)
        else:
            # captured extend: the tokens of each sequence are all new (the reference
            # approximates the same way, :838-843); the grid covers num_tokens rows
            self._cg_prefix_kv_lens[:bs].zero_()
            self._cg_seq_lens[:bs].copy_(seq)
            self._cg_query_start_loc[0] = 0
            torch.cumsum(seq, dim=0, dtype=torch.int32, out=self._cg_query_start_loc[1: bs + 1])
            mode, max_q = MODE_EXTEND, int(num_tokens)
        md = MI355XForwardMetadata(
            mode=mode, table=self.req_to_token, row_index=self._cg_row_index[:bs],
            seq_lens=self._cg_seq_lens[:bs], query_start_loc=self._cg_query_start_loc[: bs + 1],
            prefix_kv_lens=self._cg_prefix_kv_lens[:bs], causal=True, max_q_per_seq=max_q,
            num_tokens=int(num_tokens))
        if self._cg_swa_table is not None:
            md.swa_table = self._swa_rows(self._cg_row_index[:bs], md.seq_lens, out=self._cg_swa_table)[:bs]
            md.swa_row_index = torch.arange(bs, dtype=torch.int64, device=self.device)
        self.forward_metadata = md

    def init_forward_metadata_capture_cuda_graph(self, bs, num_tokens, req_pool_indices, seq_lens,
                                                 encoder_lens, forward_mode, spec_info) -> None:
        self._fill_graph_metadata(bs, num_tokens, req_pool_indices, seq_lens, forward_mode, spec_info)

    def init_forward_metadata_replay_cuda_graph(self, bs, req_pool_indices, seq_lens, seq_lens_sum,
                                                encoder_lens, forward_mode, spec_info,
                                                seq_lens_cpu=None) -> None:
        num_tokens = self.forward_metadata.num_tokens if self.forward_metadata is not None else bs
        draft = _mode_is(forward_mode, "is_draft_extend_v2") or _mode_is(forward_mode, "is_draft_extend")
        if draft and self.forward_metadata is not None and self._cg_rows_per_req:
            num_tokens = bs * self._cg_rows_per_req
        if _mode_is(forward_mode, "is_target_verify"):
            num_tokens = bs * int(spec_info.draft_token_num)
        elif _mode_is(forward_mode, "is_decode_or_idle"):
            num_tokens = bs
        self._fill_graph_metadata(bs, num_tokens, req_pool_indices, seq_lens, forward_mode, spec_info)

    def init_forward_metadata_out_graph(self, forward_batch, in_capture: bool = False) -> None:
        if in_capture:
            self.init_forward_metadata_capture_cuda_graph(
                forward_batch.batch_size, forward_batch.input_ids.shape[0], forward_batch.req_pool_indices,
                forward_batch.seq_lens, getattr(forward_batch, "encoder_lens", None),
                forward_batch.forward_mode, forward_batch.spec_info)
        else:
            self.init_forward_metadata_replay_cuda_graph(
                forward_batch.batch_size, forward_batch.req_pool_indices, forward_batch.seq_lens,
                getattr(forward_batch, "seq_lens_sum", None), getattr(forward_batch, "encoder_lens", None),
                forward_batch.forward_mode, forward_batch.spec_info,
                getattr(forward_batch, "seq_lens_cpu", None))

    # ------------------------------------------------------------------
    # Forward
    # ------------------------------------------------------------------
    def _check_layer(self, layer, kwargs) -> None:
        reason = layer_shape_reason(layer)
        if reason is None and kwargs.get("sinks") is not None:
            reason = "attention_sinks"
        if reason is not None:
            raise NotImplementedError(f"mi355x_attn cannot serve layer {getattr(layer, 'layer_id', '?')}: {reason}")

    @staticmethod
    def _scales(layer) -> tuple[float, float]:
        ks = float(layer.k_scale_float) if getattr(layer, "k_scale", None) is not None else 1.0
        vs = float(layer.v_scale_float) if getattr(layer, "v_scale", None) is not None else 1.0
        return ks, vs

    def _caches(self, layer):
        pool = self.token_to_kv_pool
        return pool.get_key_buffer(layer.layer_id), pool.get_value_buffer(layer.layer_id)

    def _kernel_q(self, q: torch.Tensor, cache_dtype: torch.dtype) -> torch.Tensor:
        """The kernels take q in the 16-bit dtype of a 16-bit cache (any 16-bit q for fp8)."""
        if cache_dtype in FP8_KV or cache_dtype == q.dtype:
            return q
        return q.to(cache_dtype)

    def _table_for(self, md: MI355XForwardMetadata, window: int):
        if window >= 0 and md.swa_table is not None:
            return md.swa_table, md.swa_row_index
        return md.table, md.row_index

    def _save_kv(self, layer, loc, k, v) -> None:
        if k is None:
            return
        # an SWA pool maps full-pool slots to its own for its sliding-window layers inside
        # its set_kv_buffer; the native write is for pools that store at the slots given
        if not self.native_kv_write or self._has_swa_pool():
            self.token_to_kv_pool.set_kv_buffer(layer, loc, k, v, layer.k_scale, layer.v_scale)
            return
        k_cache, v_cache = self._caches(layer)
        ks = float(layer.k_scale_float) if getattr(layer, "k_scale", None) is not None else None
        vs = float(layer.v_scale_float) if getattr(layer, "v_scale", None) is not None else None
        hkv, d = int(layer.tp_k_head_num), int(layer.head_dim)
        ops.set_kv_buffer(k_cache, v_cache, loc, k.reshape(-1, hkv, d), v.reshape(-1, hkv, d), ks, vs)

    def forward_decode(self, q, k, v, layer, forward_batch, save_kv_cache: bool = True, **kwargs):
        self._check_layer(layer, kwargs)
        md = self.forward_metadata
        if md is None or md.mode != MODE_DECODE:
            raise RuntimeError("forward_decode without decode metadata (init_forward_metadata first)")
        if save_kv_cache:
            self._save_kv(layer, forward_batch.out_cache_loc, k, v)
        hq, d = int(layer.tp_q_head_num), int(layer.head_dim)
        out_dtype = q.dtype
        k_cache, v_cache = self._caches(layer)
        q3 = self._kernel_q(q.reshape(-1, hq, d), k_cache.dtype)
        out = torch.empty(q3.shape, dtype=q3.dtype, device=q3.device)
        causal, window = resolve_layer_mask(
            default_causal=True, is_cross_attention=bool(getattr(layer, "is_cross_attention", False)),
            is_encoder_only=_is_encoder_only(layer),
            sliding_window_size=getattr(layer, "sliding_window_size", None))
        if q3.shape[0]:
            table, rows = self._table_for(md, window)
            ks, vs = self._scales(layer)
            ops.grouped_decode_forward(
                q3, k_cache, v_cache, table, md.seq_lens, softmax_scale=float(layer.scaling),
                k_scale=ks, v_scale=vs, out=out, row_index=rows, page_size=1,
                sliding_window_size=window, max_seq_len_hint=md.max_seq_len,
                workspace=self.splitkv_workspace())
        out = out.reshape(q3.shape[0], hq * d)
        return out if out.dtype == out_dtype else out.to(out_dtype)

    def forward_extend(self, q, k, v, layer, forward_batch, save_kv_cache: bool = True, **kwargs):
        self._check_layer(layer, kwargs)
        md = self.forward_metadata
        if md is None or md.mode == MODE_DECODE:
            raise RuntimeError("forward_extend without extend metadata (init_forward_metadata first)")
        if save_kv_cache:
            self._save_kv(layer, forward_batch.out_cache_loc, k, v)
        hq, d = int(layer.tp_q_head_num), int(layer.head_dim)
        out_dtype = q.dtype
        k_cache, v_cache = self._caches(layer)
        q3 = self._kernel_q(q.reshape(-1, hq, d), k_cache.dtype)
        out = torch.empty(q3.shape, dtype=q3.dtype, device=q3.device)
        causal, window = resolve_layer_mask(
            default_causal=md.causal, is_cross_attention=bool(getattr(layer, "is_cross_attention", False)),
            is_encoder_only=_is_encoder_only(layer),
            sliding_window_size=getattr(layer, "sliding_window_size", None))
        if q3.shape[0]:
            table, rows = self._table_for(md, window)
            ks, vs = self._scales(layer)
            ops.paged_forward(  # returns (out, softmax_lse); out is written in place
                q3, k_cache, v_cache, table, md.seq_lens, md.query_start_loc, md.prefix_kv_lens,
                out=out, block_size=1, num_kv_heads=int(layer.tp_k_head_num),
                softmax_scale=float(layer.scaling), causal=causal, sliding_window_size=window,
                linear_verify=md.mode == MODE_VERIFY, k_scale=ks, v_scale=vs, row_index=rows,
                max_q_len_hint=md.max_q_per_seq if md.mode == MODE_VERIFY else None,
                workspace=self._workspace_for(md.mode, q3.shape[0], hq, int(layer.tp_k_head_num),
                                              md.seq_lens.shape[0]))
        out = out.reshape(q3.shape[0], hq * d)
        return out if out.dtype == out_dtype else out.to(out_dtype)

    def forward(self, q, k, v, layer, forward_batch, save_kv_cache: bool = True, **kwargs):
        """Dispatch by forward mode (what the engine's base class does)."""
        if _mode_is(forward_batch.forward_mode, "is_decode_or_idle"):
            return self.forward_decode(q, k, v, layer, forward_batch, save_kv_cache=save_kv_cache, **kwargs)
        return self.forward_extend(q, k, v, layer, forward_batch, save_kv_cache=save_kv_cache, **kwargs)
