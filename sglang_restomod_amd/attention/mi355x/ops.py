"""Operators over the HIP library, with the reference adapter's signatures.

* ``grouped_decode_forward`` - sglang_restomod/attention/v100/tilelang/_paged_adapter.py:402-486
* ``paged_forward``          - _paged_adapter.py:567-759 (extend, and the linear-verify branch)
* ``set_kv_buffer``          - the token pool's write called at flash_attn_v100_backend.py:1174-1182
* ``gather_fp8_paged_kv``    - _paged_adapter.py:527-564
* ``translate_slots``        - the SWA page-table build, flash_attn_v100_backend.py:460-503
* ``draft_table``            - the draft container's per-step KV rows, draft_decode.py:172-208

Shapes and dtypes are validated here and raise ``ValueError`` the way the
reference's gates do (_paged_adapter.py:417-418, 538-541). Workspaces are
allocated by this layer (one growable buffer per device and stream, so reuse is
ordered by the stream), never by the library. Nothing here synchronises with
the host unless the caller leaves out a length hint the grid needs.
"""

from __future__ import annotations

import math
import os
from typing import Optional

import torch

from . import _lib

FP8_DTYPES = (torch.float8_e4m3fn, torch.float8_e5m2)

VERIFY_MAX_Q_PER_SEQ = 64
TUNED_HEAD_DIMS = (64, 128, 256)  # split-KV decode/verify and tiled extend kernels
MAX_HEAD_DIM = 512                 # other multiples of 16 up to this: the any-head-dim kernel
HEAD_DIM_MULTIPLE = 16


# A decode with at most this many 32-key split-KV tiles (over every sequence, kv head and
# 32-row group, at the caller's length bound) runs as key pieces on the any-head-dim kernel
# (MA_SMALL_DECODE_TILES in csrc/splitkv.hip).
SMALL_DECODE_TILES = 16384


def decode_kernel(batch: int, num_q_heads: int, num_kv_heads: int, head_dim: int,
                  max_seq_len_hint: Optional[int]) -> str:
    """Which kernel carries a decode call: ``"splitkv_partial"`` (the persistent split-KV
    kernel) or ``"any_kernel"`` (head dims other than 64/128/256, and small decodes given a
    length bound). The library makes the same choice."""
    if int(head_dim) not in TUNED_HEAD_DIMS:
        return "any_kernel"
    if not max_seq_len_hint or max_seq_len_hint <= 0:
        return "splitkv_partial"
    group = int(num_q_heads) // int(num_kv_heads)
    tiles = int(batch) * int(num_kv_heads) * ((group + 31) // 32) * ((int(max_seq_len_hint) + 31) // 32)
    return "any_kernel" if tiles <= SMALL_DECODE_TILES else "splitkv_partial"


def head_dim_supported(head_dim: int) -> bool:
    """Head dims the library serves: every multiple of 16 from 16 to 512 (64, 128 and 256 on
    the tuned kernels, the rest on the any-head-dim kernel, which needs no workspace)."""
    d = int(head_dim)
    return HEAD_DIM_MULTIPLE <= d <= MAX_HEAD_DIM and d % HEAD_DIM_MULTIPLE == 0

_WORKSPACES: dict = {}
_DEVICE_WORKGROUPS: dict = {}


def _env_int(name: str, default: int) -> int:
    raw = os.environ.get(name)
    if raw is None or not raw.strip():
        return default
    try:
        value = int(raw)
    except ValueError as exc:
        raise ValueError(f"{name} must be a positive integer") from exc
    if value <= 0:
        raise ValueError(f"{name} must be a positive integer")
    return value


def splitkv_workgroups(device: torch.device) -> int:
    """Persistent grid size of the split-KV kernels: one workgroup per compute unit
    (``SGLANG_MI355X_SPLITKV_WORKGROUPS`` overrides)."""
    key = device.index if device.index is not None else torch.cuda.current_device()
    n = _DEVICE_WORKGROUPS.get(key)
    if n is None:  # once per device: the count and the override (read at the first call)
        with torch.cuda.device(device):
            n = int(_lib.load().ma_device_workgroups())
        if n <= 0:
            raise RuntimeError("could not query the device's compute-unit count")
        n = _env_int("SGLANG_MI355X_SPLITKV_WORKGROUPS", n)
        _DEVICE_WORKGROUPS[key] = n
    return n


def q_dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.float16:
        return _lib.MA_DT_F16
    if dtype == torch.bfloat16:
        return _lib.MA_DT_BF16
    raise ValueError(f"query dtype must be float16 or bfloat16, got {dtype}")


def kv_dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.float8_e4m3fn:
        return _lib.MA_DT_E4M3
    if dtype == torch.float8_e5m2:
        return _lib.MA_DT_E5M2
    return q_dtype_code(dtype)


def kv_layout(cache: torch.Tensor, page_size: Optional[int] = None):
    """(row_stride, head_stride, page_size, num_kv_heads, head_dim) of a token pool.

    Accepts the flat pool [slots, Hkv, D] or the paged view [pages, ps, Hkv, D]
    (whose pages must be contiguous runs of rows).
    """
    st, shape = cache.stride(), cache.shape
    if len(st) == 3:
        ps = 1 if page_size is None else int(page_size)
        row, head = st[0], st[1]
        hkv, dim = shape[1], shape[2]
    elif len(st) == 4:
        ps = shape[1]
        if page_size is not None and int(page_size) != ps:
            raise ValueError(f"page_size {page_size} does not match the cache's page dim {ps}")
        if st[0] != ps * st[1]:
            raise ValueError("paged KV cache must store each page as a contiguous run of rows")
        row, head = st[1], st[2]
        hkv, dim = shape[2], shape[3]
    else:
        raise ValueError(f"KV cache must be 3-D or 4-D, got shape {tuple(shape)}")
    if st[-1] != 1:
        raise ValueError("KV cache head_dim must be contiguous")
    if ps <= 0 or ps & (ps - 1):
        raise ValueError(f"page size must be a power of two, got {ps}")
    return row, head, ps, hkv, dim


def _check_device(*tensors: torch.Tensor) -> torch.device:
    dev = tensors[0].device
    if dev.type != "cuda":
        raise ValueError("the MI355X attention operators need device tensors (got a CPU tensor)")
    for t in tensors[1:]:
        if t is not None and t.device != dev:
            raise ValueError("all operands must be on the same device")
    return dev


# The raw handle of a device's current stream, without building a Stream object (about
# 0.2 against 1.9 us per call, which matters for a decode step of about 10 us).
_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream_ptr(device: torch.device) -> int:
    if _RAW_STREAM is not None:
        return _RAW_STREAM(device.index if device.index is not None else torch.cuda.current_device())
    return torch.cuda.current_stream(device).cuda_stream


def _i64(t: Optional[torch.Tensor]) -> Optional[torch.Tensor]:
    if t is None or (t.dtype == torch.int64 and t.is_contiguous()):
        return t
    return t.to(torch.int64).contiguous()


def workspace_buffer(device: torch.device, nbytes: int, stream: Optional[int] = None) -> torch.Tensor:
    """A growable byte buffer per (device, stream), shared by the entry points that take a
    workspace; calls on one stream are ordered, so they can share it. ``stream``: the
    current stream's handle when the caller already has it."""
    if nbytes <= 0:
        return None
    key = (str(device), _stream_ptr(device) if stream is None else stream)
    buf = _WORKSPACES.get(key)
    if buf is None or buf.numel() < nbytes:
        cap = 1 << max(20, (nbytes - 1).bit_length())
        buf = torch.zeros(cap, dtype=torch.uint8, device=device)
        _WORKSPACES[key] = buf
    return buf


def splitkv_workspace_bytes(device: torch.device, head_dim: int, num_workgroups: Optional[int] = None) -> int:
    """Bytes of a split-KV workspace at this grid and head dim (0 for the head dims served
    by the any-head-dim kernel)."""
    nwg = int(num_workgroups) if num_workgroups else splitkv_workgroups(device)
    return int(_lib.load().ma_splitkv_workspace_bytes(nwg, int(head_dim)))


def splitkv_workspace(device: torch.device, num_workgroups: Optional[int] = None,
                      head_dim: int = 128) -> torch.Tensor:
    """A fresh workspace sized for the split-KV entry points at this grid (callers that
    capture graphs keep one for the graph's lifetime instead of the shared buffer)."""
    nwg = int(num_workgroups) if num_workgroups else splitkv_workgroups(device)
    nbytes = _lib.load().ma_splitkv_workspace_bytes(nwg, head_dim)
    return torch.zeros(max(nbytes, 1), dtype=torch.uint8, device=device)


_SPLITKV_WS_BYTES: dict = {}


def _splitkv_ws(lib, dev, nwg: int, D: int, given: Optional[torch.Tensor], stream: Optional[int] = None):
    nbytes = _SPLITKV_WS_BYTES.get((nwg, D))
    if nbytes is None:
        nbytes = _SPLITKV_WS_BYTES[(nwg, D)] = int(lib.ma_splitkv_workspace_bytes(nwg, D))
    if given is None:
        return workspace_buffer(dev, nbytes, stream), nbytes
    if given.dtype != torch.uint8 or given.device != dev or given.numel() < nbytes:
        raise ValueError(f"workspace must be a uint8 tensor of at least {nbytes} bytes on {dev}")
    return given, nbytes


def extend_workspace_bytes(num_tokens: int, num_q_heads: int, num_kv_heads: int, batch: int) -> int:
    """Bytes of the work list of an extend call (``ma_extend_workspace_bytes``)."""
    return int(_lib.load().ma_extend_workspace_bytes(int(num_tokens), int(num_q_heads), int(num_kv_heads),
                                                      int(batch)))


def extend_workspace(device: torch.device, num_tokens: int, num_q_heads: int, num_kv_heads: int,
                     batch: int) -> torch.Tensor:
    """A fresh workspace for ``paged_extend_forward`` calls of up to ``num_tokens`` query
    tokens in ``batch`` sequences (callers that capture graphs keep one)."""
    nbytes = extend_workspace_bytes(num_tokens, num_q_heads, num_kv_heads, batch)
    return torch.empty(max(nbytes, 1), dtype=torch.uint8, device=device)


def _i32(t: torch.Tensor) -> torch.Tensor:
    return t if (t.dtype == torch.int32 and t.is_contiguous()) else t.to(torch.int32).contiguous()


def _table(table: torch.Tensor) -> torch.Tensor:
    if table.dtype != torch.int32:
        raise ValueError(f"page table / req_to_token must be int32, got {table.dtype}")
    st = table.stride()
    if len(st) != 2 or st[1] != 1:
        raise ValueError("page table must be 2-D with contiguous rows")
    return table


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _out_code(out: torch.Tensor, q: torch.Tensor) -> int:
    """dtype code of an attention output: q's dtype, or float32 for the result before its
    rounding to 16 bits."""
    if out.shape != q.shape or out.dtype not in (q.dtype, torch.float32):
        raise ValueError("out must have q's shape, and q's dtype or float32")
    return _lib.MA_DT_F32 if out.dtype == torch.float32 else q_dtype_code(q.dtype)


def grouped_decode_forward(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    page_table: torch.Tensor,
    seq_lens: torch.Tensor,
    *,
    softmax_scale: float,
    k_scale: float = 1.0,
    v_scale: float = 1.0,
    out: Optional[torch.Tensor] = None,
    row_index: Optional[torch.Tensor] = None,
    page_size: Optional[int] = None,
    sliding_window_size: int = -1,
    max_seq_len_hint: Optional[int] = None,
    num_workgroups: Optional[int] = None,
    workspace: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Decode one query token per sequence: ``q`` [B, Hq, D] -> [B, Hq, D] in q's dtype, or
    in float32 when ``out`` is float32 (the result before its rounding to 16 bits).

    ``page_table`` [rows, width] int32 maps (row, position // page_size) to a page;
    ``row_index`` [B] picks each sequence's row (None: row b). With page size 1
    and ``req_to_token`` / ``req_pool_indices`` this reads SGLang's slots directly.
    ``workspace``: a uint8 buffer from ``splitkv_workspace`` (None: a shared buffer
    per device and stream).
    """
    if q.dim() != 3:
        raise ValueError(f"q must be [batch, heads, head_dim], got {tuple(q.shape)}")
    if v_cache.dtype != k_cache.dtype:
        raise ValueError("K and V cache dtypes must match for grouped decode.")
    dev = _check_device(q, k_cache, v_cache, page_table, seq_lens, row_index)
    B, Hq, D = q.shape
    row, head, ps, Hkv, Dk = kv_layout(k_cache, page_size)
    if v_cache.stride() != k_cache.stride():  # equal strides: the same layout
        vrow, vhead, _, _, _ = kv_layout(v_cache, ps)
        if (vrow, vhead) != (row, head):
            raise ValueError("K and V caches must share one layout")
    if Dk != D:
        raise ValueError(f"head_dim mismatch: q {D}, cache {Dk}")
    if Hq % Hkv:
        raise ValueError(f"query heads {Hq} must be a multiple of kv heads {Hkv}")
    if q.stride(-1) != 1:
        q = q.contiguous()
    table = _table(page_table)
    if out is None:
        out = torch.empty_like(q, memory_format=torch.contiguous_format)
    out_code = _out_code(out, q)
    seq = _i32(seq_lens)
    ridx = _i64(row_index)
    # a host-known bound of the lengths picks the single-pass path for small batches; it
    # never changes the result
    max_len = 0 if max_seq_len_hint is None else max(0, int(max_seq_len_hint))
    nwg = int(num_workgroups) if num_workgroups else splitkv_workgroups(dev)
    lib = _lib.load()
    stream = _stream_ptr(dev)
    ws, nbytes = _splitkv_ws(lib, dev, nwg, D, workspace, stream)
    qs, os_ = q.stride(), out.stride()
    status = lib.ma_grouped_decode(
        q.data_ptr(), qs[0], qs[1], q_dtype_code(q.dtype),
        k_cache.data_ptr(), v_cache.data_ptr(), row, head, kv_dtype_code(k_cache.dtype),
        table.data_ptr(), table.stride()[0], _ptr(ridx), ps,
        seq.data_ptr(), B, Hq, Hkv, D,
        nwg, float(softmax_scale), float(k_scale), float(v_scale),
        int(sliding_window_size), max_len, _ptr(ws), nbytes,
        out.data_ptr(), out_code, os_[0], os_[1], stream,
    )
    _lib.check(status, "ma_grouped_decode")
    return out


def paged_verify_forward(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_table: torch.Tensor,
    seq_lens: torch.Tensor,
    query_start_loc: torch.Tensor,
    prefix_kv_lens: Optional[torch.Tensor],
    *,
    max_q_per_seq: int,
    softmax_scale: float,
    k_scale: float = 1.0,
    v_scale: float = 1.0,
    causal: bool = True,
    sliding_window_size: int = -1,
    out: Optional[torch.Tensor] = None,
    row_index: Optional[torch.Tensor] = None,
    page_size: Optional[int] = None,
    max_seq_len_hint: Optional[int] = None,
    num_workgroups: Optional[int] = None,
    workspace: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Few query rows per sequence over a long prefix (linear-chain target verify).

    ``max_q_per_seq`` is the longest chain expected: it picks the kernel's row-group
    shape. Every query row of every sequence is computed whatever the hint says."""
    if q.dim() != 3:
        raise ValueError(f"q must be [tokens, heads, head_dim], got {tuple(q.shape)}")
    if v_cache.dtype != k_cache.dtype:
        raise ValueError("K and V cache dtypes must match")
    dev = _check_device(q, k_cache, v_cache, block_table, seq_lens, query_start_loc)
    T, Hq, D = q.shape
    row, head, ps, Hkv, Dk = kv_layout(k_cache, page_size)
    if kv_layout(v_cache, ps)[:2] != (row, head):
        raise ValueError("K and V caches must share one layout")
    if Dk != D or Hq % Hkv:
        raise ValueError("head shape mismatch between q and the KV cache")
    if not 0 < max_q_per_seq <= VERIFY_MAX_Q_PER_SEQ:
        raise ValueError(f"the verify hint must be 1..{VERIFY_MAX_Q_PER_SEQ} query rows per sequence")
    if q.stride(-1) != 1:
        q = q.contiguous()
    table = _table(block_table)
    B = seq_lens.shape[0]
    if out is None:
        out = torch.empty_like(q, memory_format=torch.contiguous_format)
    out_code = _out_code(out, q)
    seq = _i32(seq_lens)
    qsl = _i32(query_start_loc)
    pre = None if prefix_kv_lens is None else _i32(prefix_kv_lens)
    ridx = _i64(row_index)
    del max_seq_len_hint
    nwg = int(num_workgroups) if num_workgroups else splitkv_workgroups(dev)
    lib = _lib.load()
    stream = _stream_ptr(dev)
    ws, nbytes = _splitkv_ws(lib, dev, nwg, D, workspace, stream)
    status = lib.ma_paged_verify(
        q.data_ptr(), q.stride(0), q.stride(1), q_dtype_code(q.dtype), T,
        k_cache.data_ptr(), v_cache.data_ptr(), row, head, kv_dtype_code(k_cache.dtype),
        table.data_ptr(), table.stride(0), _ptr(ridx), ps,
        seq.data_ptr(), qsl.data_ptr(), _ptr(pre),
        B, int(max_q_per_seq), Hq, Hkv, D,
        1 if causal else 0, int(sliding_window_size), nwg,
        float(softmax_scale), float(k_scale), float(v_scale), _ptr(ws), nbytes,
        out.data_ptr(), out_code, out.stride(0), out.stride(1), stream,
    )
    _lib.check(status, "ma_paged_verify")
    return out


def paged_forward(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_table: torch.Tensor,
    seq_lens: torch.Tensor,
    query_start_loc: torch.Tensor,
    prefix_kv_lens: torch.Tensor,
    out: Optional[torch.Tensor] = None,
    block_size: Optional[int] = 16,
    num_kv_heads: Optional[int] = None,
    softmax_scale: Optional[float] = None,
    causal: bool = True,
    sliding_window_size: int = -1,
    linear_verify: bool = False,
    k_scale: float = 1.0,
    v_scale: float = 1.0,
    max_seq_len_hint: Optional[int] = None,
    logical_dense_kv: bool = False,
    row_index: Optional[torch.Tensor] = None,
    max_q_len_hint: Optional[int] = None,
    workspace: Optional[torch.Tensor] = None,
):
    """Prefix-aware paged attention over ``q`` [num_tokens, Hq, D] (reference: paged_forward,
    _paged_adapter.py:567-759, same positional arguments). Returns ``(out, softmax_lse)``
    as the reference does (:756-759); ``softmax_lse`` is an fp32 ``[Hq, num_tokens]``
    buffer that, as in the reference, is allocated and not filled.

    ``block_size`` is the page size of ``block_table`` (default 16, the reference's): a
    4-D cache ``[pages, page_size, Hkv, D]`` must agree with it; a flat pool
    ``[slots, Hkv, D]`` is read as pages of ``block_size`` rows (``block_size=1`` with
    ``req_to_token`` / ``row_index`` addresses SGLang's token pool directly).
    ``linear_verify`` sends batches with at most ``VERIFY_MAX_Q_PER_SEQ`` query rows per
    sequence on average (a bound from the shapes alone, as the reference routes,
    :613-617) to the split-KV verifier; ``max_q_len_hint`` (the longest chain) only
    picks its row-group shape. No host value of the device tensors is read.
    ``logical_dense_kv`` is accepted for signature compatibility; it changes no result.
    """
    del logical_dense_kv
    T, Hq, D = q.shape
    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(D)
    if block_size is not None and k_cache.dim() == 4 and int(block_size) != k_cache.shape[1]:
        raise ValueError(f"block_size {block_size} does not match the cache's page dim {k_cache.shape[1]}")
    if num_kv_heads is not None:
        hkv = kv_layout(k_cache, block_size)[3]
        if hkv != int(num_kv_heads):
            raise ValueError(f"num_kv_heads {num_kv_heads} does not match the cache ({hkv})")
    B = seq_lens.shape[0]
    lse = torch.empty(Hq, T, dtype=torch.float32, device=q.device)
    if linear_verify and B > 0 and T <= B * VERIFY_MAX_Q_PER_SEQ:
        hint = int(max_q_len_hint) if max_q_len_hint else min(T, VERIFY_MAX_Q_PER_SEQ)
        hint = max(1, min(hint, VERIFY_MAX_Q_PER_SEQ))
        out = paged_verify_forward(
            q, k_cache, v_cache, block_table, seq_lens, query_start_loc, prefix_kv_lens,
            max_q_per_seq=hint, softmax_scale=softmax_scale, k_scale=k_scale, v_scale=v_scale,
            causal=causal, sliding_window_size=sliding_window_size, out=out, row_index=row_index,
            page_size=block_size, max_seq_len_hint=max_seq_len_hint, workspace=workspace)
        return out, lse
    out = paged_extend_forward(
        q, k_cache, v_cache, block_table, seq_lens, query_start_loc, prefix_kv_lens,
        softmax_scale=softmax_scale, k_scale=k_scale, v_scale=v_scale,
        causal=causal, sliding_window_size=sliding_window_size, out=out, row_index=row_index,
        page_size=block_size, workspace=workspace)
    return out, lse


def paged_extend_forward(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_table: torch.Tensor,
    seq_lens: torch.Tensor,
    query_start_loc: torch.Tensor,
    prefix_kv_lens: Optional[torch.Tensor],
    *,
    softmax_scale: float,
    k_scale: float = 1.0,
    v_scale: float = 1.0,
    causal: bool = True,
    sliding_window_size: int = -1,
    out: Optional[torch.Tensor] = None,
    row_index: Optional[torch.Tensor] = None,
    page_size: Optional[int] = None,
    workspace: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Prefix-aware extend on MFMA tiles: ``q`` [num_tokens, Hq, D] -> ``out`` (q's dtype).

    The row tiles are listed on the device, so no host value of the query lengths is
    read. ``workspace`` (uint8, ``extend_workspace``) defaults to the shared buffer of
    the current stream; a split-KV workspace of enough bytes serves as well."""
    if q.dim() != 3:
        raise ValueError(f"q must be [tokens, heads, head_dim], got {tuple(q.shape)}")
    if v_cache.dtype != k_cache.dtype:
        raise ValueError("K and V cache dtypes must match")
    dev = _check_device(q, k_cache, v_cache, block_table, seq_lens, query_start_loc)
    T, Hq, D = q.shape
    row, head, ps, Hkv, Dk = kv_layout(k_cache, page_size)
    if kv_layout(v_cache, ps)[:2] != (row, head):
        raise ValueError("K and V caches must share one layout")
    if Dk != D or Hq % Hkv:
        raise ValueError("head shape mismatch between q and the KV cache")
    if q.stride(-1) != 1:
        q = q.contiguous()
    table = _table(block_table)
    if out is None:
        out = torch.empty_like(q, memory_format=torch.contiguous_format)
    out_code = _out_code(out, q)
    B = seq_lens.shape[0]
    seq = _i32(seq_lens)
    qsl = _i32(query_start_loc)
    pre = None if prefix_kv_lens is None else _i32(prefix_kv_lens)
    ridx = _i64(row_index)
    lib = _lib.load()
    nbytes = lib.ma_extend_workspace_bytes(T, Hq, Hkv, B)
    stream = _stream_ptr(dev)
    if workspace is None:
        ws = workspace_buffer(dev, nbytes, stream)
    else:
        if workspace.dtype != torch.uint8 or workspace.device != dev or workspace.numel() < nbytes:
            raise ValueError(f"workspace must be a uint8 tensor of at least {nbytes} bytes on {dev}")
        ws = workspace
    status = lib.ma_paged_extend(
        q.data_ptr(), q.stride(0), q.stride(1), q_dtype_code(q.dtype), T,
        k_cache.data_ptr(), v_cache.data_ptr(), row, head, kv_dtype_code(k_cache.dtype),
        table.data_ptr(), table.stride(0), _ptr(ridx), ps,
        seq.data_ptr(), qsl.data_ptr(), _ptr(pre),
        B, Hq, Hkv, D, 1 if causal else 0, int(sliding_window_size),
        float(softmax_scale), float(k_scale), float(v_scale), _ptr(ws), nbytes,
        out.data_ptr(), out_code, out.stride(0), out.stride(1), stream,
    )
    _lib.check(status, "ma_paged_extend")
    return out


def set_kv_buffer(
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    loc: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    k_scale: Optional[float] = None,
    v_scale: Optional[float] = None,
) -> None:
    """Store new K/V rows ``k``/``v`` [T, Hkv, D] at pool slots ``loc`` [T] (the token
    pool's ``set_kv_buffer``): a copy into a pool of the source dtype; otherwise, with
    scales given, ``x / scale`` rounded to the source dtype, then cast to the pool dtype
    (fp8: round to nearest even, e4m3fn overflow -> NaN, e5m2 overflow -> inf).
    Pools are [slots, Hkv, D] (or the paged view); slots outside the pool are skipped.
    """
    if k.dim() == 2:
        k = k.view(k.shape[0], -1, k_cache.shape[-1])
        v = v.view(v.shape[0], -1, v_cache.shape[-1])
    if k.shape != v.shape or k.dim() != 3:
        raise ValueError("k and v must be [tokens, kv_heads, head_dim] of one shape")
    if k.dtype != v.dtype or k_cache.dtype != v_cache.dtype:
        raise ValueError("k/v and the two caches must share their dtypes")
    dev = _check_device(k, v, k_cache, v_cache, loc)
    T, H, D = k.shape
    row, head, ps, Hc, Dc = kv_layout(k_cache)
    if kv_layout(v_cache)[:2] != (row, head):
        raise ValueError("K and V caches must share one layout")
    if (Hc, Dc) != (H, D):
        raise ValueError(f"cache heads/dim {(Hc, Dc)} do not match the rows {(H, D)}")
    if k.stride() != v.stride() or k.stride(-1) != 1:
        k, v = k.contiguous(), v.contiguous()
    slots = k_cache.shape[0] * (ps if k_cache.dim() == 4 else 1)
    loc64 = loc.to(torch.int64).contiguous()
    apply = k_cache.dtype != k.dtype and k_scale is not None
    ks = float(k_scale) if apply else 1.0
    vs = float(v_scale) if (apply and v_scale is not None) else (1.0 if not apply else ks)
    status = _lib.load().ma_set_kv_buffer(
        k.data_ptr(), v.data_ptr(), k.stride(0), k.stride(1), q_dtype_code(k.dtype),
        loc64.data_ptr(), T, H, D,
        k_cache.data_ptr(), v_cache.data_ptr(), row, head, kv_dtype_code(k_cache.dtype),
        slots, ks, vs, 1 if apply else 0, _stream_ptr(dev),
    )
    _lib.check(status, "ma_set_kv_buffer")


def translate_slots(
    table: torch.Tensor,
    seq_lens: torch.Tensor,
    mapping: torch.Tensor,
    row_index: Optional[torch.Tensor] = None,
    out: Optional[torch.Tensor] = None,
    width: Optional[int] = None,
) -> torch.Tensor:
    """Rows of ``table`` (req_to_token, int32) translated through ``mapping`` (the SWA
    pool's ``full_to_swa_index_mapping``), on the device: ``out[b, j] =
    mapping[table[row_index[b], j]]`` for ``j < seq_lens[b]``; slots outside the mapping
    give 0 and positions from ``seq_lens[b]`` on are left as they are. ``out`` defaults to
    a new ``[B, width]`` int32 tensor, ``width`` to the table's width; no host value of
    the lengths is read."""
    if table.dtype != torch.int32 or table.dim() != 2 or table.stride(1) != 1:
        raise ValueError("table must be a 2-D int32 tensor with contiguous rows")
    dev = _check_device(table, seq_lens, mapping)
    B = int(seq_lens.shape[0])
    width = int(table.shape[1] if width is None else width)
    if width > table.shape[1]:
        raise ValueError(f"width {width} exceeds the table's {table.shape[1]} columns")
    if out is None:
        out = torch.empty(B, width, dtype=torch.int32, device=dev)
    if out.dtype != torch.int32 or out.dim() != 2 or out.stride(1) != 1 or out.shape[0] < B or out.shape[1] < width:
        raise ValueError(f"out must be an int32 [>= {B}, >= {width}] tensor with contiguous rows")
    seq = _i32(seq_lens)
    m64 = mapping if (mapping.dtype == torch.int64 and mapping.is_contiguous()) else mapping.to(torch.int64).contiguous()
    ridx = _i64(row_index)
    status = _lib.load().ma_translate_slots(
        table.data_ptr(), table.stride(0), _ptr(ridx), seq.data_ptr(), B, m64.data_ptr(), m64.numel(),
        out.data_ptr(), out.stride(0), width, _stream_ptr(dev))
    _lib.check(status, "ma_translate_slots")
    return out


def draft_table(
    table: torch.Tensor,
    seq_lens: torch.Tensor,
    topk: int,
    num_steps: int,
    row_index: Optional[torch.Tensor] = None,
    mapping: Optional[torch.Tensor] = None,
    out: Optional[torch.Tensor] = None,
    width: Optional[int] = None,
) -> torch.Tensor:
    """Key rows of a multi-step draft (``ma_draft_table``): row ``b * topk + k`` holds the
    prefix slots of request ``b`` (``table[row_index[b], :seq_lens[b]]``) followed by
    branch ``k``'s ``num_steps`` draft slots, which sit at ``seq_lens[b] + k * num_steps``
    of the request's row. ``mapping`` (an SWA pool's full-to-SWA index) translates every
    slot. ``out`` defaults to a new ``[B * topk, width]`` int32 tensor (``width``: the
    table's); entries past each row's ``seq_lens[b] + num_steps`` are left as they are."""
    if table.dtype != torch.int32 or table.dim() != 2 or table.stride(1) != 1:
        raise ValueError("table must be a 2-D int32 tensor with contiguous rows")
    if topk <= 0 or num_steps <= 0:
        raise ValueError(f"topk ({topk}) and num_steps ({num_steps}) must be positive")
    dev = _check_device(table, seq_lens, row_index, mapping)
    B = int(seq_lens.shape[0])
    rows = B * int(topk)
    width = int(table.shape[1] if width is None else width)
    if out is None:
        out = torch.empty(rows, width, dtype=torch.int32, device=dev)
    if out.dtype != torch.int32 or out.dim() != 2 or out.stride(1) != 1 or out.shape[0] < rows or out.shape[1] < width:
        raise ValueError(f"out must be an int32 [>= {rows}, >= {width}] tensor with contiguous rows")
    seq = _i32(seq_lens)
    ridx = _i64(row_index)
    m64 = None
    if mapping is not None:
        m64 = mapping if (mapping.dtype == torch.int64 and mapping.is_contiguous()) else mapping.to(torch.int64).contiguous()
    status = _lib.load().ma_draft_table(
        table.data_ptr(), table.stride(0), int(table.shape[1]), _ptr(ridx), seq.data_ptr(), B, int(topk),
        int(num_steps), _ptr(m64), 0 if m64 is None else m64.numel(), out.data_ptr(), out.stride(0), width,
        _stream_ptr(dev))
    _lib.check(status, "ma_draft_table")
    return out


def gather_fp8_paged_kv(k_cache, v_cache, page_table, seq_lens, k_output, v_output) -> None:
    """Resolve and decode the logical fp8 pages of each sequence into caller-owned fp16
    buffers (reference: gather_fp8_paged_kv, same arguments and errors): caches
    [num_pages, page_size, Hkv, D] in e4m3fn or e5m2, page_table [B, max_blocks],
    outputs [B * max_blocks, page_size, Hkv, D] fp16; logical page p of sequence b
    (p < ceil(seq_lens[b] / page_size)) goes to output page b * max_blocks + p."""
    if k_cache.dtype not in FP8_DTYPES:
        raise ValueError("gather_fp8_paged_kv expects E4M3 or E5M2 cache")
    if v_cache.dtype != k_cache.dtype:
        raise ValueError("K and V cache dtypes must match")
    if k_cache.dim() != 4 or v_cache.shape != k_cache.shape or k_cache.stride() != v_cache.stride():
        raise ValueError("caches must be [pages, page_size, heads, head_dim] of one layout")
    if k_cache.stride(3) != 1:
        raise ValueError("head_dim must be contiguous in the caches")
    dev = _check_device(k_cache, v_cache, page_table, seq_lens, k_output, v_output)
    num_pages, ps, hkv, d = k_cache.shape
    B, max_blocks = page_table.shape
    want = (B * max_blocks, ps, hkv, d)
    for o in (k_output, v_output):
        if tuple(o.shape) != want or o.dtype != torch.float16 or not o.is_contiguous():
            raise ValueError(f"outputs must be contiguous float16 {want}")
    table = _i32(page_table)
    seq = _i32(seq_lens)
    status = _lib.load().ma_gather_fp8_paged_kv(
        k_cache.data_ptr(), v_cache.data_ptr(), k_cache.stride(0), k_cache.stride(1), k_cache.stride(2),
        kv_dtype_code(k_cache.dtype), num_pages, table.data_ptr(), table.stride(0), seq.data_ptr(),
        B, max_blocks, ps, hkv, d, k_output.data_ptr(), v_output.data_ptr(), _stream_ptr(dev))
    _lib.check(status, "ma_gather_fp8_paged_kv")
