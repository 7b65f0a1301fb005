"""Loader for libmi355x_attn.so (the C ABI declared in include/mi355x_attn.h).

torch is imported first on purpose: it ships its own HIP runtime with the same
soname (libamdhip64.so.7), and loading it first makes the library bind to that
one copy, so device pointers and streams are shared with torch.

There is no fallback: if the library is missing or fails to load, every
operator raises.
"""

from __future__ import annotations

import ctypes
import os
import threading
from ctypes import c_float, c_int, c_int64, c_size_t, c_void_p, c_char_p

_LOCK = threading.Lock()
_LIB = None

LIB_PATH = os.path.join(os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__)))),
                        "libmi355x_attn.so")

MA_DT_F16, MA_DT_BF16, MA_DT_E4M3, MA_DT_E5M2, MA_DT_F32 = 0, 1, 2, 3, 4
MA_OK = 0
MA_EINVAL, MA_ELAUNCH, MA_EUNSUPPORTED = -1, -2, -3
# grid limit of ma_grouped_decode_noalloc's static scratch (include/mi355x_attn.h)
MA_NOALLOC_MAX_WORKGROUPS = 256

# name -> (restype, argtypes); the header is the source of truth.
SIGNATURES = {
    "ma_last_error": (c_char_p, []),
    "ma_abi_version": (c_int, []),
    "ma_device_arch": (c_int, [c_char_p, c_int]),
    "ma_device_workgroups": (c_int, []),
    "ma_splitkv_workspace_bytes": (c_size_t, [c_int, c_int]),
    "ma_grouped_decode": (c_int, [
        c_void_p, c_int64, c_int64, c_int,            # q, strides, dtype
        c_void_p, c_void_p, c_int64, c_int64, c_int,  # k, v, row/head stride, kv dtype
        c_void_p, c_int64, c_void_p, c_int,           # table, stride, row_index, page size
        c_void_p, c_int, c_int, c_int, c_int,         # seq_lens, batch, hq, hkv, dim
        c_int, c_float, c_float, c_float,             # num_workgroups, scales
        c_int, c_int, c_void_p, c_size_t,             # window, max_seq_len, workspace, bytes
        c_void_p, c_int, c_int64, c_int64, c_void_p,  # out, out dtype, strides, stream
    ]),
    "ma_grouped_decode_noalloc": (c_int, [
        c_void_p, c_int64, c_int64, c_int,            # q, strides, dtype
        c_void_p, c_void_p, c_int64, c_int64, c_int,  # k, v, row/head stride, kv dtype
        c_void_p, c_int64, c_void_p, c_int,           # table, stride, row_index, page size
        c_void_p, c_int, c_int, c_int, c_int,         # seq_lens, batch, hq, hkv, dim
        c_int, c_float, c_float, c_float, c_int,      # num_workgroups, scales, window
        c_int,                                        # max_seq_len
        c_void_p, c_int, c_int64, c_int64, c_void_p,  # out, out dtype, strides, stream
    ]),
    "ma_paged_verify": (c_int, [
        c_void_p, c_int64, c_int64, c_int, c_int64,   # q, strides, dtype, num_tokens
        c_void_p, c_void_p, c_int64, c_int64, c_int,  # k, v, strides, kv dtype
        c_void_p, c_int64, c_void_p, c_int,           # table, stride, row_index, page size
        c_void_p, c_void_p, c_void_p,                 # seq_lens, qsl, prefix
        c_int, c_int, c_int, c_int, c_int,            # batch, max_q, hq, hkv, dim
        c_int, c_int, c_int,                          # causal, window, num_workgroups
        c_float, c_float, c_float, c_void_p, c_size_t,  # scales, workspace, bytes
        c_void_p, c_int, c_int64, c_int64, c_void_p,  # out, out dtype, strides, stream
    ]),
    "ma_set_kv_buffer": (c_int, [
        c_void_p, c_void_p, c_int64, c_int64, c_int,  # k, v, strides, source dtype
        c_void_p, c_int64, c_int, c_int,              # loc, num_tokens, hkv, dim
        c_void_p, c_void_p, c_int64, c_int64, c_int,  # caches, strides, cache dtype
        c_int64, c_float, c_float, c_int, c_void_p,   # num_slots, scales, apply, stream
    ]),
    "ma_translate_slots": (c_int, [
        c_void_p, c_int64, c_void_p, c_void_p, c_int,  # table, stride, row_index, seq_lens, batch
        c_void_p, c_int64,                            # mapping, mapping_len
        c_void_p, c_int64, c_int, c_void_p,           # out, stride, width, stream
    ]),
    "ma_draft_table": (c_int, [
        c_void_p, c_int64, c_int, c_void_p,           # table, stride, width, row_index
        c_void_p, c_int, c_int, c_int,                # seq_lens, batch, topk, num_steps
        c_void_p, c_int64,                            # mapping, mapping_len
        c_void_p, c_int64, c_int, c_void_p,           # out, stride, width, stream
    ]),
    "ma_gather_fp8_paged_kv": (c_int, [
        c_void_p, c_void_p, c_int64, c_int64, c_int64,  # caches, page/token/head strides (bytes)
        c_int, c_int64, c_void_p, c_int64, c_void_p,  # dtype, num_pages, page_table, stride, seq_lens
        c_int, c_int, c_int, c_int, c_int,            # batch, max_blocks, page_size, hkv, dim
        c_void_p, c_void_p, c_void_p,                 # k_out, v_out, stream
    ]),
    "ma_extend_workspace_bytes": (c_size_t, [c_int64, c_int, c_int, c_int]),
    "ma_paged_extend": (c_int, [
        c_void_p, c_int64, c_int64, c_int, c_int64,   # q, strides, dtype, num_tokens
        c_void_p, c_void_p, c_int64, c_int64, c_int,  # k, v, strides, kv dtype
        c_void_p, c_int64, c_void_p, c_int,           # table, stride, row_index, page size
        c_void_p, c_void_p, c_void_p,                 # seq_lens, qsl, prefix
        c_int, c_int, c_int, c_int,                   # batch, hq, hkv, dim
        c_int, c_int, c_float, c_float, c_float,      # causal, window, scales
        c_void_p, c_size_t,                           # workspace, bytes
        c_void_p, c_int, c_int64, c_int64, c_void_p,  # out, out dtype, strides, stream
    ]),
}


class LibraryError(RuntimeError):
    pass


def load():
    """Load (once) and return the ctypes library; raise if it is missing."""
    global _LIB
    if _LIB is not None:
        return _LIB
    with _LOCK:
        if _LIB is not None:
            return _LIB
        import torch  # noqa: F401  (binds the library to torch's HIP runtime)

        if not os.path.exists(LIB_PATH):
            raise LibraryError(
                f"{LIB_PATH} is not built; run `python -m sglang_restomod_amd.build` "
                "(there is no CPU or PyTorch fallback for the MI355X attention backend)"
            )
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = lib
        return lib


def check(status: int, what: str) -> None:
    if status != MA_OK:
        msg = load().ma_last_error().decode(errors="replace")
        if status == -1:
            raise ValueError(f"{what}: {msg}")
        raise RuntimeError(f"{what} failed ({status}): {msg}")
