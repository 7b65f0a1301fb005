"""End-to-end through MI355XAttnBackend on the GPU: a serving sequence over the
fake engine (cached prefix -> extend -> decode -> linear verify -> draft extend)
for each KV dtype (and at head dims 64 and 256 for bf16 and e4m3), and decode
captured in a HIP graph and replayed with new lengths. Every output is checked against the float64 oracle over the pool as the
backend left it (after its own K/V writes)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import attention as oracle
from tests import fakes
from tests.helpers import assert_attn_close, to_f64

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
HQ, HKV, D = 16, 2, 128


def _backend(engine):
    from sglang_restomod_amd.attention.mi355x.backend import MI355XAttnBackend

    return MI355XAttnBackend(engine.runner)


def _layer(kv_dtype, hq=HQ, hkv=HKV, dim=D):
    shape = dict(head_dim=dim, scaling=dim ** -0.5)
    if kv_dtype in fakes.FP8:
        return fakes.Layer(hq, hkv, k_scale=torch.tensor(1.5, device=DEV), v_scale=torch.tensor(0.75, device=DEV),
                           k_scale_float=1.5, v_scale_float=0.75, **shape)
    return fakes.Layer(hq, hkv, **shape)


def _pools(eng):
    k = eng.pool.get_key_buffer(0)
    v = eng.pool.get_value_buffer(0)
    return to_f64(k), to_f64(v)


def _check_extend(eng, layer, fb, q, out, prefix, ext, what):
    hq, dim = layer.tp_q_head_num, layer.head_dim
    kp, vp = _pools(eng)
    r2t = eng.req_to_token.cpu().numpy()
    rows = fb.req_pool_indices.tolist()
    ref = oracle.extend(to_f64(q).reshape(-1, hq, dim), kp, vp, r2t, rows, prefix, ext,
                        softmax_scale=layer.scaling, k_scale=layer.k_scale_float, v_scale=layer.v_scale_float)
    assert out.shape == q.shape and out.dtype == q.dtype
    assert_attn_close(out.reshape(-1, hq, dim), ref, what=what)


def _rand(gen, *shape, dtype=torch.bfloat16):
    return torch.randn(*shape, generator=gen).to(dtype).to(DEV)


def _serving_sequence(kv_dtype, HQ=HQ, HKV=HKV, D=D, page_size=1):
    print(f"[case] serving sequence {kv_dtype} hq={HQ} hkv={HKV} d={D} page_size={page_size}", flush=True)
    gen = torch.Generator().manual_seed(7)
    eng = fakes.Engine(DEV, hq=HQ, hkv=HKV, head_dim=D, kv_dtype=kv_dtype, pool_size=12000, max_reqs=6,
                       context_len=4096, spec="EAGLE", topk=1, page_size=page_size)
    layer = _layer(kv_dtype, HQ, HKV, D)
    be = _backend(eng)
    # cached prefixes computed by earlier forwards
    prefix = {0: 300, 1: 0, 2: 1000}
    for r, p in prefix.items():
        if p:
            slots = eng.alloc(r, p)
            eng.fill(0, slots, _rand(gen, p, HKV, D), _rand(gen, p, HKV, D), layer)
    rows = [0, 1, 2]
    # extend (chunked prefill over the cached prefix)
    ext = [77, 130, 5]
    fb = eng.batch("EXTEND", rows, new_tokens=ext)
    T = sum(ext)
    q, k, v = _rand(gen, T, HQ * D), _rand(gen, T, HKV, D), _rand(gen, T, HKV, D)
    be.init_forward_metadata(fb)
    out = be.forward_extend(q, k, v, layer, fb)
    _check_extend(eng, layer, fb, q, out, [prefix[r] for r in rows], ext, f"extend {kv_dtype}")
    # two decode steps, batch order differing from request order
    for step in range(2):
        fb = eng.batch("DECODE", [2, 0, 1], new_tokens=[1, 1, 1])
        q, k, v = _rand(gen, 3, HQ * D), _rand(gen, 3, HKV, D), _rand(gen, 3, HKV, D)
        be.init_forward_metadata(fb)
        out = be.forward_decode(q, k, v, layer, fb)
        kp, vp = _pools(eng)
        ref = oracle.decode(to_f64(q).reshape(3, HQ, D), kp, vp, eng.req_to_token.cpu().numpy(), [2, 0, 1],
                            fb.seq_lens.tolist(), softmax_scale=layer.scaling, k_scale=layer.k_scale_float,
                            v_scale=layer.v_scale_float)
        assert out.shape == (3, HQ * D) and out.dtype == q.dtype
        assert_attn_close(out.reshape(3, HQ, D), ref, what=f"decode step {step} {kv_dtype}")
    # linear target verify: 4 draft tokens per request over the whole context
    fb = eng.batch("TARGET_VERIFY", rows, new_tokens=[4, 4, 4], draft_token_num=4)
    q, k, v = _rand(gen, 12, HQ * D), _rand(gen, 12, HKV, D), _rand(gen, 12, HKV, D)
    be.init_forward_metadata(fb)
    assert be.forward_metadata.mode == "verify"
    out = be.forward_extend(q, k, v, layer, fb)
    _check_extend(eng, layer, fb, q, out, fb.before, [4, 4, 4], f"verify {kv_dtype}")
    # draft extend: a few rows per request, served by the verify kernel
    fb = eng.batch("DRAFT_EXTEND_V2", rows, new_tokens=[3, 1, 6])
    q, k, v = _rand(gen, 10, HQ * D), _rand(gen, 10, HKV, D), _rand(gen, 10, HKV, D)
    be.init_forward_metadata(fb)
    assert be.forward_metadata.mode == "verify"
    out = be.forward_extend(q, k, v, layer, fb)
    _check_extend(eng, layer, fb, q, out, fb.before, [3, 1, 6], f"draft extend {kv_dtype}")


@pytest.mark.parametrize("kv_dtype", [torch.bfloat16, torch.float16, torch.float8_e4m3fn, torch.float8_e5m2])
def test_serving_sequence(kv_dtype):
    _serving_sequence(kv_dtype)


@pytest.mark.parametrize("kv_dtype", [torch.bfloat16, torch.float8_e4m3fn])
@pytest.mark.parametrize("hq,hkv,dim", [(8, 2, 64), (12, 2, 256), (8, 2, 96), (8, 2, 192), (8, 2, 80),
                                        (16, 4, 512)])
def test_serving_sequence_head_dims(kv_dtype, hq, hkv, dim):
    """The same sequence at head dims 64 and 256 (the latter with the 27B model's
    per-GPU head counts); at 96 and 192, whose extend runs on the padded tiled kernels
    that skip their zero steps, and 80, padded without the skip; and at 512. Decode and
    verify at the dims other than 64/128/256 run on the any-head-dim kernel."""
    _serving_sequence(kv_dtype, hq, hkv, dim)


@pytest.mark.parametrize("kv_dtype", [torch.bfloat16, torch.float8_e4m3fn])
def test_serving_sequence_page_size_16(kv_dtype):
    """The same sequence on an engine with 16-token pages (the reference's production page
    size): every request's positions sit in runs of 16 consecutive slots, and the kernels
    address them through the engine's token-level req_to_token."""
    _serving_sequence(kv_dtype, page_size=16)


def test_sliding_window_layer_through_swa_pool():
    gen = torch.Generator().manual_seed(11)
    eng = fakes.Engine(DEV, hq=HQ, hkv=HKV, kv_dtype=torch.bfloat16, pool_size=6000, max_reqs=4,
                       context_len=2048, swa=True)
    full = fakes.Layer(HQ, HKV, layer_id=0)
    be = _backend(eng)
    rows = [0, 1]
    fb = eng.batch("EXTEND", rows, new_tokens=[400, 90])
    T = 490
    q, k, v = _rand(gen, T, HQ * D), _rand(gen, T, HKV, D), _rand(gen, T, HKV, D)
    be.init_forward_metadata(fb)
    # the SWA layer's K/V live at the translated slots of the same pool (a stand-in for
    # the separate SWA pool): write them there, then attend through the swa table
    swa = fakes.Layer(HQ, HKV, layer_id=0, sliding_window_size=64)
    eng.pool.set_kv_buffer(swa, fb.out_cache_loc, k, v)  # the pool maps them to SWA slots
    out = be.forward_extend(q, k, v, swa, fb, save_kv_cache=False)
    kp, vp = _pools(eng)
    swa_r2t = eng.pool.full_to_swa_index_mapping[eng.req_to_token.long()].cpu().numpy()
    ref = oracle.extend(to_f64(q).reshape(-1, HQ, D), kp, vp, swa_r2t, rows, [0, 0], [400, 90],
                        softmax_scale=swa.scaling, sliding_window=64)
    assert_attn_close(out.reshape(-1, HQ, D), ref, what="swa extend")
    del full


@pytest.mark.parametrize("HQ,HKV,D", [(HQ, HKV, D), (8, 2, 96), (16, 4, 512)])
def test_decode_in_a_hip_graph_replays_with_new_lengths(HQ, HKV, D):
    """At head dims 96 and 512 the decode runs on the any-head-dim kernel (no workspace)."""
    print(f"[case] decode graph hq={HQ} hkv={HKV} d={D}", flush=True)
    gen = torch.Generator().manual_seed(3)
    eng = fakes.Engine(DEV, hq=HQ, hkv=HKV, head_dim=D, kv_dtype=torch.bfloat16, pool_size=9000, max_reqs=8,
                       context_len=4096)
    layer = _layer(torch.bfloat16, HQ, HKV, D)
    be = _backend(eng)
    rows = [4, 1, 6, 0]
    for r, n in zip(rows, [700, 33, 1500, 260]):
        s = eng.alloc(r, n)
        eng.fill(0, s, _rand(gen, n, HKV, D), _rand(gen, n, HKV, D), layer)
    bs = len(rows)
    be.init_cuda_graph_state(max_bs=8, max_num_tokens=8)
    fb = eng.batch("DECODE", rows, new_tokens=[1] * bs)
    eng.fill(0, fb.out_cache_loc, _rand(gen, bs, HKV, D), _rand(gen, bs, HKV, D), layer)
    q_static = _rand(gen, bs, HQ * D)
    be.init_forward_metadata_capture_cuda_graph(bs, bs, fb.req_pool_indices, fb.seq_lens, None,
                                                fb.forward_mode, None)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        be.forward_decode(q_static, None, None, layer, fb, save_kv_cache=False)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_static = be.forward_decode(q_static, None, None, layer, fb, save_kv_cache=False)
    for step in range(4):
        # grow every request by one token (step 3 re-runs the same lengths)
        if step < 3:
            fb = eng.batch("DECODE", rows, new_tokens=[1] * bs)
            eng.fill(0, fb.out_cache_loc, _rand(gen, bs, HKV, D), _rand(gen, bs, HKV, D), layer)
        q_static.copy_(_rand(gen, bs, HQ * D))
        be.init_forward_metadata_replay_cuda_graph(bs, fb.req_pool_indices, fb.seq_lens, fb.seq_lens_sum,
                                                   None, fb.forward_mode, None, fb.seq_lens_cpu)
        graph.replay()
        torch.cuda.synchronize()
        got = out_static.clone()
        # eager runs of the same batch between replays: without the host's length bound
        # (the kernels the graph captured, bit for bit), and with it (the eager path, which
        # may take the key pieces)
        be.init_forward_metadata(fb)
        hinted = be.forward_decode(q_static, None, None, layer, fb, save_kv_cache=False)
        be.forward_metadata.max_seq_len = 0
        eager = be.forward_decode(q_static, None, None, layer, fb, save_kv_cache=False)
        torch.cuda.synchronize()
        assert torch.equal(got, eager), f"replay {step} differs from the eager call"
        kp, vp = _pools(eng)
        ref = oracle.decode(to_f64(q_static).reshape(bs, HQ, D), kp, vp, eng.req_to_token.cpu().numpy(), rows,
                            fb.seq_lens.tolist(), softmax_scale=layer.scaling)
        assert_attn_close(got.reshape(bs, HQ, D), ref, what=f"graph replay {step}")
        assert_attn_close(hinted.reshape(bs, HQ, D), ref, what=f"eager with the length bound {step}")


@pytest.mark.parametrize("mode", ["DRAFT_EXTEND_V2", "DRAFT_EXTEND"])
def test_draft_extend_in_a_hip_graph_replays_with_new_lengths(mode):
    """A draft extend captured with three rows per request, replayed over grown requests:
    every replay equals the eager call on the same batch and the float64 oracle."""
    print(f"[case] draft extend graph {mode}", flush=True)
    gen = torch.Generator().manual_seed(5)
    eng = fakes.Engine(DEV, hq=HQ, hkv=HKV, kv_dtype=torch.bfloat16, pool_size=9000, max_reqs=8,
                       context_len=4096, spec="EAGLE", draft_worker=True)
    layer = _layer(torch.bfloat16)
    be = _backend(eng)
    rows, n = [5, 2, 7], 3
    for r, p in zip(rows, [900, 40, 1700]):
        s = eng.alloc(r, p)
        eng.fill(0, s, _rand(gen, p, HKV, D), _rand(gen, p, HKV, D), layer)
    bs = len(rows)
    be.init_cuda_graph_state(max_bs=8, max_num_tokens=8 * n)
    fb = eng.batch(mode, rows, new_tokens=[n] * bs)
    eng.fill(0, fb.out_cache_loc, _rand(gen, bs * n, HKV, D), _rand(gen, bs * n, HKV, D), layer)
    q_static = _rand(gen, bs * n, HQ * D)
    be.init_forward_metadata_capture_cuda_graph(bs, bs * n, fb.req_pool_indices, fb.seq_lens, None,
                                                fb.forward_mode, None)
    assert be.forward_metadata.mode == "verify"
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        be.forward_extend(q_static, None, None, layer, fb, save_kv_cache=False)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_static = be.forward_extend(q_static, None, None, layer, fb, save_kv_cache=False)
    for step in range(3):
        if step < 2:  # the next round's rows (step 2 replays the same lengths)
            fb = eng.batch(mode, rows, new_tokens=[n] * bs)
            eng.fill(0, fb.out_cache_loc, _rand(gen, bs * n, HKV, D), _rand(gen, bs * n, HKV, D), layer)
        q_static.copy_(_rand(gen, bs * n, HQ * D))
        be.init_forward_metadata_replay_cuda_graph(bs, fb.req_pool_indices, fb.seq_lens, fb.seq_lens_sum,
                                                   None, fb.forward_mode, None, fb.seq_lens_cpu)
        graph.replay()
        torch.cuda.synchronize()
        got = out_static.clone()
        be.init_forward_metadata(fb)
        eager = be.forward_extend(q_static, None, None, layer, fb, save_kv_cache=False)
        torch.cuda.synchronize()
        assert torch.equal(got, eager), f"replay {step} differs from the eager call"
        _check_extend(eng, layer, fb, q_static, got, fb.before, [n] * bs, f"draft extend replay {step}")


@pytest.mark.parametrize("kv_dtype", [torch.bfloat16, torch.float8_e4m3fn, torch.float8_e5m2])
def test_native_kv_write_matches_the_pool_write(kv_dtype, monkeypatch):
    """The library's KV write leaves the pool byte-identical to the pool's own write."""
    engines, outs = [], []
    for native in (False, True):
        monkeypatch.setenv("SGLANG_MI355X_NATIVE_KV_WRITE", "1" if native else "0")
        gen = torch.Generator().manual_seed(21)
        eng = fakes.Engine(DEV, hq=HQ, hkv=HKV, kv_dtype=kv_dtype, pool_size=4000, max_reqs=4, context_len=2048)
        layer = _layer(kv_dtype)
        be = _backend(eng)
        assert be.native_kv_write == native
        fb = eng.batch("EXTEND", [0, 1], new_tokens=[150, 40])
        q, k, v = _rand(gen, 190, HQ * D), _rand(gen, 190, HKV, D), _rand(gen, 190, HKV, D)
        be.init_forward_metadata(fb)
        o1 = be.forward_extend(q, k, v, layer, fb)
        fb = eng.batch("DECODE", [1, 0], new_tokens=[1, 1])
        q, k, v = _rand(gen, 2, HQ * D), _rand(gen, 2, HKV, D), _rand(gen, 2, HKV, D)
        be.init_forward_metadata(fb)
        o2 = be.forward_decode(q, k, v, layer, fb)
        torch.cuda.synchronize()
        engines.append(eng)
        outs.append((o1, o2))
    for name in ("k_buffer", "v_buffer"):
        a = getattr(engines[0].pool, name)[0]
        b = getattr(engines[1].pool, name)[0]
        assert torch.equal(a.view(torch.uint8), b.view(torch.uint8)), name
    assert engines[1].pool.writes == 0 and engines[0].pool.writes == 2
    for x, y in zip(outs[0], outs[1]):
        assert torch.equal(x, y)
