"""Decode split over key pieces (the any-head-dim kernel with one workgroup per piece of a
sequence's keys, then a merge kernel) against the float64 oracle and against the unsplit
paths on the same inputs.

* Head dims 64, 128 and 256: a decode whose split-KV work is small runs on the pieces when
  the caller passes a host-known length bound (``max_seq_len_hint``) above 512 keys (at or
  below it, on one workgroup per row block); without one it runs on the persistent
  split-KV kernel. All are checked.
* Other head dims: with a workspace, a batch that leaves compute units idle is split into
  pieces; with a grid of one workgroup (``num_workgroups=1``) it is not. Both are checked,
  including a single sequence of 32k keys at head dims 96 and 512 (the case that ran on
  one workgroup per kv head before the split).

Every case is seeded; empty sequences, one-key sequences, sliding windows, GQA groups of 1
to 16 and every KV dtype appear.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import attention as oracle
from tests.helpers import assert_attn_close, to_f64

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
FP8 = (torch.float8_e4m3fn, torch.float8_e5m2)


def _ops():
    from sglang_restomod_amd.attention.mi355x import ops

    return ops


def _build(seed, dim, lens, hkv, group, kv, window=-1):
    gen = torch.Generator().manual_seed(seed)
    B = len(lens)
    pool = sum(lens) + 8
    ks, vs = (1.25, 0.75) if kv in FP8 else (1.0, 1.0)
    kf = torch.randn(pool, hkv, dim, generator=gen)
    vf = torch.randn(pool, hkv, dim, generator=gen)
    if kv in FP8:
        k, v = (kf / ks).to(kv), (vf / vs).to(kv)
        q_dtype = torch.bfloat16
    else:
        k, v = kf.to(kv), vf.to(kv)
        q_dtype = kv
    q = torch.randn(B, hkv * group, dim, generator=gen).to(q_dtype)
    perm = torch.randperm(pool - 1, generator=gen) + 1
    rows = torch.randperm(B + 2, generator=gen)[:B]
    r2t = torch.zeros(B + 2, max(max(lens), 1) + 3, dtype=torch.int32)
    off = 0
    for b, n in enumerate(lens):
        r2t[rows[b], :n] = perm[off:off + n].to(torch.int32)
        off += n
    print(f"[case] pieces seed={seed} D={dim} lens={lens if len(lens) < 8 else len(lens)} hkv={hkv} G={group} "
          f"kv={kv} window={window}", flush=True)
    return dict(q=q.to(DEV), k=k.to(DEV), v=v.to(DEV), r2t=r2t.to(DEV), rows=rows.to(DEV), lens=lens,
                seq=torch.tensor(lens, dtype=torch.int32, device=DEV), ks=ks, vs=vs, scale=dim ** -0.5,
                window=window)


def _run(c, **kw):
    out = _ops().grouped_decode_forward(c["q"], c["k"], c["v"], c["r2t"], c["seq"], softmax_scale=c["scale"],
                                        k_scale=c["ks"], v_scale=c["vs"], row_index=c["rows"],
                                        sliding_window_size=c["window"], **kw)
    torch.cuda.synchronize()
    return out


def _gather_f64(pool, slots):
    if pool.dtype in FP8:
        return pool.view(torch.uint8)[slots].cpu().view(pool.dtype).float().numpy().astype(np.float64)
    return pool[slots].float().cpu().numpy().astype(np.float64)


def _check(c, out, what):
    r2t = c["r2t"].cpu().numpy()
    rows = c["rows"].cpu().numpy()
    q = to_f64(c["q"])
    for b, n in enumerate(c["lens"]):
        slots = torch.from_numpy(r2t[rows[b], :n].astype(np.int64)).to(DEV)
        kb, vb = _gather_f64(c["k"], slots), _gather_f64(c["v"], slots)
        table = np.arange(max(n, 1), dtype=np.int64)[None, :]
        if n == 0:
            kb = np.zeros((1,) + tuple(c["k"].shape[1:]))
            vb = np.zeros_like(kb)
        ref = oracle.decode(q[b:b + 1], kb, vb, table, [0], [n], softmax_scale=c["scale"], k_scale=c["ks"],
                            v_scale=c["vs"], sliding_window=c["window"])
        assert_attn_close(out[b:b + 1], ref, what=f"{what} seq {b} (ctx {n})")


TUNED = [
    (1, 128, [700], 8, 4, torch.float16, -1),
    (2, 128, [700, 0, 1, 33], 8, 8, torch.bfloat16, -1),
    (3, 128, [3000, 40], 2, 16, torch.float8_e4m3fn, 100),
    (4, 64, [900, 17], 4, 5, torch.float8_e5m2, -1),
    (5, 256, [1500, 2], 2, 6, torch.bfloat16, 0),
    (6, 256, [64], 1, 1, torch.float16, -1),
]


@pytest.mark.parametrize("seed,dim,lens,hkv,group,kv,window", TUNED)
def test_small_decode_runs_on_pieces_with_a_length_bound(seed, dim, lens, hkv, group, kv, window):
    c = _build(seed, dim, lens, hkv, group, kv, window)
    split = _run(c, max_seq_len_hint=max(lens))
    _check(c, split, f"pieces D={dim}")
    persistent = _run(c)
    _check(c, persistent, f"persistent D={dim}")
    # a loose bound cuts the keys into other pieces (other rounding), still within the bound
    _check(c, _run(c, max_seq_len_hint=3 * max(lens)), f"pieces, loose bound D={dim}")
    # the same bound gives the same pieces: bit-identical
    assert torch.equal(split, _run(c, max_seq_len_hint=max(lens)))


ANY = [
    (11, 96, [2000, 5, 0], 4, 4, torch.bfloat16, -1),
    (12, 192, [800, 1200], 2, 8, torch.float8_e4m3fn, -1),
    (13, 320, [900], 1, 3, torch.float16, 50),
    (14, 512, [1024, 9], 4, 4, torch.float8_e5m2, -1),
    (15, 48, [4000], 8, 2, torch.bfloat16, -1),
]


@pytest.mark.parametrize("seed,dim,lens,hkv,group,kv,window", ANY)
def test_any_head_dim_decode_splits_keys_over_pieces(seed, dim, lens, hkv, group, kv, window):
    c = _build(seed, dim, lens, hkv, group, kv, window)
    split = _run(c, max_seq_len_hint=max(lens))
    _check(c, split, f"pieces D={dim}")
    unsplit = _run(c, num_workgroups=1)
    _check(c, unsplit, f"unsplit D={dim}")
    # without a length bound the pieces follow the table width; the result stays in bounds
    _check(c, _run(c), f"pieces by table width D={dim}")


@pytest.mark.parametrize("dim", [96, 512])
def test_single_long_sequence_at_other_head_dims(dim):
    """One sequence of 32k keys, 4 kv heads: split over pieces instead of 4 workgroups."""
    c = _build(21, dim, [32768], 4, 4, torch.bfloat16)
    _check(c, _run(c, max_seq_len_hint=32768), f"long D={dim}")


def test_pieces_in_a_hip_graph_replay_with_new_lengths():
    """A captured decode at head dim 96 (pieces chosen from the table width) replays with
    longer sequences: every replay equals the eager call and the oracle."""
    c = _build(31, 96, [600, 900], 2, 4, torch.bfloat16)
    ops = _ops()
    ws = ops.splitkv_workspace(DEV, head_dim=96)
    out = torch.empty_like(c["q"])

    def call():
        ops.grouped_decode_forward(c["q"], c["k"], c["v"], c["r2t"], c["seq"], softmax_scale=c["scale"],
                                   row_index=c["rows"], out=out, workspace=ws)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        call()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call()
    for step, lens in enumerate(([601, 901], [602, 902], [602, 902])):
        c["seq"].copy_(torch.tensor(lens, dtype=torch.int32))
        c["lens"] = lens
        graph.replay()
        torch.cuda.synchronize()
        got = out.clone()
        call()
        torch.cuda.synchronize()
        assert torch.equal(got, out), f"replay {step} differs from the eager call"
        _check(c, got, f"graph replay {step}")
