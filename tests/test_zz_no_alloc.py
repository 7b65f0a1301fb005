"""ma_grouped_decode_noalloc through the C ABI against ma_grouped_decode on the same inputs:
bit-identical outputs on two calls in a row, the second on a smaller batch (the static
scratch keeps the first call's contents), at head dims 128, 256 and 512 (the last on the
any-head-dim kernel, which uses no scratch) and with fp8 KV; a grid beyond the scratch is
refused before any launch. In a fresh process, the first call (which looks up the scratch's
address on the device) can be made inside HIP graph capture, and a warm call leaves the
device's free memory unchanged."""

from __future__ import annotations

import ctypes
import os
import subprocess
import sys
import textwrap

import pytest
import torch

from sglang_restomod_amd import workloads
from sglang_restomod_amd.attention.mi355x import _lib, ops

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def _args(w, out, nwg):
    k, v = w.k_pool, w.v_pool
    row, head, ps, hkv, dim = ops.kv_layout(k)
    seq = w.seq_lens.to(torch.int32).contiguous()
    ridx = w.req_pool_indices.to(torch.int64).contiguous()
    stream = torch.cuda.current_stream(DEV).cuda_stream
    head_args = (w.q.data_ptr(), w.q.stride(0), w.q.stride(1), ops.q_dtype_code(w.q.dtype),
                 k.data_ptr(), v.data_ptr(), row, head, ops.kv_dtype_code(k.dtype),
                 w.req_to_token.data_ptr(), w.req_to_token.stride(0), ridx.data_ptr(), ps,
                 seq.data_ptr(), w.batch, w.heads, hkv, dim, nwg,
                 ctypes.c_float(w.softmax_scale), ctypes.c_float(w.k_scale), ctypes.c_float(w.v_scale), -1,
                 max(w.seq_lens_cpu))
    tail = (out.data_ptr(), ops.q_dtype_code(out.dtype), out.stride(0), out.stride(1), stream)
    return head_args, tail, (seq, ridx)


def _both(w, nwg):
    lib = _lib.load()
    want = torch.empty_like(w.q)
    got = torch.full_like(w.q, float("nan"))
    head, tail, keep = _args(w, want, nwg)
    ws = ops.splitkv_workspace(DEV, num_workgroups=nwg, head_dim=w.dim)
    rc = lib.ma_grouped_decode(*head, ws.data_ptr(), ws.numel(), *tail)
    assert rc == 0, lib.ma_last_error()
    head, tail, keep2 = _args(w, got, nwg)
    rc = lib.ma_grouped_decode_noalloc(*head, *tail)
    assert rc == 0, lib.ma_last_error()
    torch.cuda.synchronize()
    del keep, keep2
    return want, got


@pytest.mark.parametrize("index,kv_format,dim", [(1, "e4m3", 128), (3, "e5m2", 128), (5, "e4m3", 256),
                                                 (7, "e4m3", 512)])
def test_noalloc_matches_the_workspace_entry_point(index, kv_format, dim):
    nwg = min(ops.splitkv_workgroups(DEV), _lib.MA_NOALLOC_MAX_WORKGROUPS)
    for call, (batch, scale) in enumerate(((24, 0.5), (5, 0.1))):  # the second call is smaller
        print(f"[case] noalloc workload {index} {kv_format} call {call} batch {batch}", flush=True)
        w = workloads.make(index, device=DEV, batch=batch, scale_lens=scale, kv_format=kv_format)
        assert w.dim == dim
        want, got = _both(w, nwg)
        assert torch.equal(want, got), f"call {call}: outputs differ"


def test_noalloc_refuses_a_grid_beyond_its_scratch():
    w = workloads.make(1, device=DEV, batch=2, scale_lens=0.05)
    lib = _lib.load()
    out = torch.empty_like(w.q)
    head, tail, keep = _args(w, out, _lib.MA_NOALLOC_MAX_WORKGROUPS + 1)
    rc = lib.ma_grouped_decode_noalloc(*head, *tail)
    assert rc == _lib.MA_EINVAL
    assert b"static scratch" in lib.ma_last_error()
    del keep


_FIRST_CALL_IN_CAPTURE = textwrap.dedent("""
    import ctypes, sys, torch
    sys.path.insert(0, {root!r})
    from sglang_restomod_amd import workloads
    from sglang_restomod_amd.attention.mi355x import _lib, ops
    from tests.test_zz_no_alloc import _args
    dev = torch.device("cuda:0")
    lib = _lib.load()
    nwg = min(ops.splitkv_workgroups(dev), _lib.MA_NOALLOC_MAX_WORKGROUPS)
    w = workloads.make(1, device=dev, batch=6, scale_lens=0.2)
    got = torch.full_like(w.q, float("nan"))
    head, tail, keep = _args(w, got, nwg)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):   # the process's first noalloc call: scratch lookup inside capture
        rc = lib.ma_grouped_decode_noalloc(*head, *tail)
    assert rc == 0, lib.ma_last_error()
    for _ in range(3):
        g.replay()
    torch.cuda.synchronize()
    want = torch.empty_like(w.q)
    h2, t2, keep2 = _args(w, want, nwg)
    ws = ops.splitkv_workspace(dev, num_workgroups=nwg, head_dim=w.dim)
    assert lib.ma_grouped_decode(*h2, ws.data_ptr(), ws.numel(), *t2) == 0, lib.ma_last_error()
    torch.cuda.synchronize()
    assert torch.equal(got, want), "graph replay differs from the workspace entry point"
    # a warm call allocates nothing: the device's free memory is unchanged
    free0 = torch.cuda.mem_get_info(dev)[0]
    assert lib.ma_grouped_decode_noalloc(*head, *tail) == 0
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info(dev)[0] == free0, "a noalloc call changed the free device memory"
    print("FIRST_CALL_IN_CAPTURE_OK", flush=True)
""")


def test_noalloc_first_call_inside_graph_capture_in_a_fresh_process():
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    print("[case] noalloc first call inside capture (subprocess)", flush=True)
    proc = subprocess.run([sys.executable, "-c", _FIRST_CALL_IN_CAPTURE.format(root=root)], cwd=root,
                          capture_output=True, text=True, timeout=180)
    assert proc.returncode == 0 and "FIRST_CALL_IN_CAPTURE_OK" in proc.stdout, (proc.stdout[-2000:],
                                                                                proc.stderr[-3000:])
