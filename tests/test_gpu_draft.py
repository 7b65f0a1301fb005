"""A draft step on the GPU: split-KV decode over the step's flat kv_indptr /
kv_indices list (ragged rows, shared prefixes as with top-k branches, an empty row),
eagerly and from a captured HIP graph, against the float64 oracle, at 16 query heads on 4
kv heads with D=128 and at the reference draft kernel's layout (6 on 1, D=256)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import attention as oracle
from tests import fakes
from tests.helpers import assert_attn_close, to_f64

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
HQ, HKV, D = 16, 4, 128


def _rand(gen, *shape):
    return torch.randn(*shape, generator=gen).to(torch.bfloat16).to(DEV)


def _lists(eng, rows_tokens):
    """kv_indptr / kv_indices for rows given as lists of slots."""
    indptr = [0]
    for toks in rows_tokens:
        indptr.append(indptr[-1] + len(toks))
    flat = [s for toks in rows_tokens for s in toks]
    return (torch.tensor(indptr, dtype=torch.int32, device=DEV),
            torch.tensor(flat, dtype=torch.int32, device=DEV))


def _reference(eng, layer, q, rows_tokens):
    kp = to_f64(eng.pool.get_key_buffer(0))
    vp = to_f64(eng.pool.get_value_buffer(0))
    slots = [np.asarray(t, dtype=np.int64) for t in rows_tokens]
    n = [len(t) for t in rows_tokens]
    hq, dim = layer.tp_q_head_num, layer.head_dim
    return oracle.paged_attention(to_f64(q).reshape(len(n), hq, dim), kp, vp, slots, list(range(len(n) + 1)),
                                  [max(x - 1, 0) for x in n], n, softmax_scale=layer.scaling,
                                  k_scale=layer.k_scale_float, v_scale=layer.v_scale_float)


def _step(eng, topk=2):
    from sglang_restomod_amd.attention.mi355x.draft_decode import MI355XDraftDecodeBackend

    return MI355XDraftDecodeBackend(eng.runner, topk, 4096, 1, 3)


@pytest.mark.parametrize("kv_dtype", [torch.bfloat16, torch.float8_e5m2])
@pytest.mark.parametrize("HQ,HKV,D", [(HQ, HKV, D), (6, 1, 256)])
def test_draft_step_over_flat_index_lists(kv_dtype, HQ, HKV, D):
    """(6, 1, 256) is the head layout of the reference's draft-decode kernel
    (sm70_longctx_decode.cu, H6/D256)."""
    print(f"[case] draft step {kv_dtype} hq={HQ} hkv={HKV} d={D}", flush=True)
    gen = torch.Generator().manual_seed(13)
    eng = fakes.Engine(DEV, hq=HQ, hkv=HKV, head_dim=D, kv_dtype=kv_dtype, pool_size=6000, max_reqs=4,
                       context_len=4096)
    shape = dict(head_dim=D, scaling=D ** -0.5)
    layer = (fakes.Layer(HQ, HKV, k_scale=torch.tensor(1.25), v_scale=torch.tensor(0.5), k_scale_float=1.25,
                         v_scale_float=0.5, **shape) if kv_dtype != torch.bfloat16 else fakes.Layer(HQ, HKV, **shape))
    prefix = {}
    for r, n in ((0, 900), (1, 37), (2, 2000)):
        s = eng.alloc(r, n)
        eng.fill(0, s, _rand(gen, n, HKV, D), _rand(gen, n, HKV, D), layer)
        prefix[r] = eng.req_to_token[r, :n].tolist()
    # draft rows: two branches of request 0 (top-k 2), request 1, request 2, and a row
    # whose list is empty
    new = [eng.free.pop() for _ in range(4)]
    rows = [prefix[0] + [new[0]], prefix[0] + [new[1]], prefix[1] + [new[2]], prefix[2] + [new[3]], []]
    rows_with_token = rows[:4]
    indptr, indices = _lists(eng, rows)
    step = _step(eng)
    assert step.refresh(indptr, indices) == 5
    q = _rand(gen, 5, HQ * D)
    k, v = _rand(gen, 4, HKV, D), _rand(gen, 4, HKV, D)
    fb = type("FB", (), {})()
    fb.out_cache_loc = torch.tensor(new, dtype=torch.int64, device=DEV)
    # the row without keys has no new token: write the four tokens first, then attend
    eng.pool.set_kv_buffer(layer, fb.out_cache_loc, k, v, layer.k_scale, layer.v_scale)
    out = step.forward_decode(q, None, None, layer, fb, save_kv_cache=False)
    torch.cuda.synchronize()
    ref = _reference(eng, layer, q, rows)
    assert out.shape == (5, HQ * D)
    assert_attn_close(out.reshape(5, HQ, D), ref, what=f"draft step {kv_dtype}")
    assert float(out[4].abs().max()) == 0.0  # no keys: zeros
    del rows_with_token


@pytest.mark.parametrize("HQ,HKV,D", [(HQ, HKV, D), (6, 1, 256)])
def test_draft_step_in_a_hip_graph(HQ, HKV, D):
    gen = torch.Generator().manual_seed(17)
    print(f"[case] draft graph hq={HQ} hkv={HKV} d={D}", flush=True)
    eng = fakes.Engine(DEV, hq=HQ, hkv=HKV, head_dim=D, kv_dtype=torch.bfloat16, pool_size=6000, max_reqs=4,
                       context_len=4096)
    layer = fakes.Layer(HQ, HKV, head_dim=D, scaling=D ** -0.5)
    base = {}
    for r, n in ((0, 300), (1, 1200)):
        s = eng.alloc(r, n)
        eng.fill(0, s, _rand(gen, n, HKV, D), _rand(gen, n, HKV, D), layer)
        base[r] = eng.req_to_token[r, :n].tolist()
    step = _step(eng, topk=1)
    step.init_cuda_graph_state(max_bs=2, max_num_tokens=2)
    cap = 4000  # fixed index buffer, as the engine's container keeps
    indptr_buf = torch.zeros(3, dtype=torch.int32, device=DEV)
    indices_buf = torch.zeros(cap, dtype=torch.int32, device=DEV)

    def fill(rows):
        ip, ix = _lists(eng, rows)
        indptr_buf.copy_(ip)
        indices_buf[:ix.numel()].copy_(ix)
        step.refresh(indptr_buf, indices_buf)

    rows = [base[0], base[1]]
    fill(rows)
    q_static = _rand(gen, 2, HQ * D)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step.forward_decode(q_static, None, None, layer, None, save_kv_cache=False)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_static = step.forward_decode(q_static, None, None, layer, None, save_kv_cache=False)
    for it in range(3):
        # every replay: one more draft token per row
        for r in (0, 1):
            s = eng.alloc(r, 1)
            eng.fill(0, s, _rand(gen, 1, HKV, D), _rand(gen, 1, HKV, D), layer)
            base[r] = eng.req_to_token[r, :eng.lens[r]].tolist()
        rows = [base[0], base[1]]
        fill(rows)
        q_static.copy_(_rand(gen, 2, HQ * D))
        graph.replay()
        torch.cuda.synchronize()
        got = out_static.clone()
        eager = step.forward_decode(q_static, None, None, layer, None, save_kv_cache=False)
        torch.cuda.synchronize()
        assert torch.equal(got, eager), f"replay {it}"
        assert_attn_close(got.reshape(2, HQ, D), _reference(eng, layer, q_static, rows), what=f"replay {it}")
