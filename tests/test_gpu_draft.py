"""Multi-step draft decode on the GPU through MI355XMultiStepDraftBackend, against the
float64 oracle:

* one pass served from a flat index list (ragged rows, two branches sharing a prefix,
  a row with no keys), at 16 query heads on 4 kv heads with D=128 and at the reference
  draft kernel's layout (6 on 1, D=256);
* whole draft rounds as the engine runs them (draft slots placed after each prefix,
  every pass writing its token's K/V, then attending): top-k 1 at page size 1 and 16,
  top-k 2, an fp8 pool, and an SWA pool with a sliding-window draft layer. The round's
  key rows (ma_draft_table) are compared bit for bit with oracle.metadata.draft_rows;
* rounds captured in a HIP graph and replayed with new lengths and new draft slots.
"""

from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from oracle import attention as oracle
from oracle import metadata as meta
from tests import fakes
from tests.helpers import assert_attn_close, pool_f64, to_f64

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
HQ, HKV, D = 16, 4, 128


def _rand(gen, *shape):
    return torch.randn(*shape, generator=gen).to(torch.bfloat16).to(DEV)


def _layer(kv_dtype, hq, hkv, dim, window=-1):
    shape = dict(head_dim=dim, scaling=dim ** -0.5, sliding_window_size=window)
    if kv_dtype in fakes.FP8:
        return fakes.Layer(hq, hkv, k_scale=torch.tensor(1.25), v_scale=torch.tensor(0.5), k_scale_float=1.25,
                           v_scale_float=0.5, **shape)
    return fakes.Layer(hq, hkv, **shape)


def _container(eng, topk, steps, layer):
    from sglang_restomod_amd.attention.mi355x.draft_decode import MI355XMultiStepDraftBackend

    eng.runner.model_config.dtype = torch.bfloat16
    return MI355XMultiStepDraftBackend(eng.runner, topk, steps, layers=[layer])


def _reference(eng, layer, q, rows_slots, swa=False):
    """Each row decodes its last key: pool read through SWA slots for an SWA layer."""
    ks = layer.k_scale_float if layer.k_scale is not None else 1.0
    vs = layer.v_scale_float if layer.v_scale is not None else 1.0
    kp = pool_f64(eng.pool.get_key_buffer(0))
    vp = pool_f64(eng.pool.get_value_buffer(0))
    mapping = eng.pool.full_to_swa_index_mapping.cpu().numpy() if swa else None
    slots = [np.asarray(t, dtype=np.int64) if mapping is None else mapping[np.asarray(t, dtype=np.int64)]
             for t in rows_slots]
    n = [len(t) for t in rows_slots]
    hq, dim = layer.tp_q_head_num, layer.head_dim
    return oracle.paged_attention(to_f64(q).reshape(len(n), hq, dim), kp, vp, slots, list(range(len(n) + 1)),
                                  [max(x - 1, 0) for x in n], n, softmax_scale=layer.scaling, k_scale=ks,
                                  v_scale=vs, sliding_window=layer.sliding_window_size)


# ---------------------------------------------------------------------------
# a pass over a flat index list
# ---------------------------------------------------------------------------
def _lists(rows_tokens):
    indptr = [0]
    for toks in rows_tokens:
        indptr.append(indptr[-1] + len(toks))
    flat = [s for toks in rows_tokens for s in toks]
    return (torch.tensor(indptr, dtype=torch.int32, device=DEV),
            torch.tensor(flat, dtype=torch.int32, device=DEV))


@pytest.mark.parametrize("kv_dtype", [torch.bfloat16, torch.float8_e5m2])
@pytest.mark.parametrize("HQ,HKV,D", [(HQ, HKV, D), (6, 1, 256)])
def test_pass_over_flat_index_lists(kv_dtype, HQ, HKV, D):
    """(6, 1, 256) is the head layout of the reference's draft-decode kernel
    (sm70_longctx_decode.cu, H6/D256)."""
    print(f"[case] draft pass over flat lists {kv_dtype} hq={HQ} hkv={HKV} d={D}", flush=True)
    gen = torch.Generator().manual_seed(13)
    eng = fakes.Engine(DEV, hq=HQ, hkv=HKV, head_dim=D, kv_dtype=kv_dtype, pool_size=6000, max_reqs=4,
                       context_len=4096)
    layer = _layer(kv_dtype, HQ, HKV, D)
    prefix = {}
    for r, n in ((0, 900), (1, 37), (2, 2000)):
        s = eng.alloc(r, n)
        eng.fill(0, s, _rand(gen, n, HKV, D), _rand(gen, n, HKV, D), layer)
        prefix[r] = eng.req_to_token[r, :n].tolist()
    # rows: two branches of request 0, request 1, request 2, and a row with no keys
    new = [eng.free.pop() for _ in range(4)]
    rows = [prefix[0] + [new[0]], prefix[0] + [new[1]], prefix[1] + [new[2]], prefix[2] + [new[3]], []]
    cont = _container(eng, 2, 2, layer)
    step = cont.attn_backends[0]
    assert step.use_flat_lists(*_lists(rows)) == 5
    q = _rand(gen, 5, HQ * D)
    k, v = _rand(gen, 4, HKV, D), _rand(gen, 4, HKV, D)
    fb = SimpleNamespace(out_cache_loc=torch.tensor(new, dtype=torch.int64, device=DEV))
    # the row without keys has no new token: write the four tokens first, then attend
    eng.pool.set_kv_buffer(layer, fb.out_cache_loc, k, v, layer.k_scale, layer.v_scale)
    out = step.forward_decode(q, None, None, layer, fb, save_kv_cache=False)
    torch.cuda.synchronize()
    assert out.shape == (5, HQ * D)
    assert_attn_close(out.reshape(5, HQ, D), _reference(eng, layer, q, rows), what=f"draft pass {kv_dtype}")
    assert float(out[4].abs().max()) == 0.0  # no keys: zeros


# ---------------------------------------------------------------------------
# whole rounds
# ---------------------------------------------------------------------------
def _engine_round(eng, reqs, topk, steps):
    """Place topk * steps draft slots after each prefix (branch k's at seq + k * steps), as
    the engine does; the committed lengths stay the prefixes."""
    seq = [eng.lens[r] for r in reqs]
    for r in reqs:
        eng.alloc(r, topk * steps)
        eng.lens[r] -= topk * steps
    fb = SimpleNamespace(req_pool_indices=torch.tensor(reqs, dtype=torch.int64, device=DEV),
                         seq_lens=torch.tensor(seq, dtype=torch.int64, device=DEV),
                         seq_lens_cpu=torch.tensor(seq), batch_size=len(reqs), spec_info=None)
    return seq, fb


def _pass_rows(eng, reqs, seq, topk, steps, i):
    """Slots each row attends over in pass i, and the slots pass i writes."""
    r2t = eng.req_to_token.cpu()
    rows, loc = [], []
    for b, r in enumerate(reqs):
        for k in range(topk):
            base = seq[b] + k * steps
            rows.append(r2t[r, :seq[b]].tolist() + r2t[r, base:base + i + 1].tolist())
            loc.append(int(r2t[r, base + i]))
    return rows, loc


ROUNDS = [
    # kv dtype, top-k, steps, page size, swa pool, draft layer window
    (torch.bfloat16, 1, 4, 1, False, -1),
    (torch.bfloat16, 1, 3, 16, False, -1),
    (torch.bfloat16, 2, 3, 1, False, -1),
    (torch.float8_e4m3fn, 2, 3, 1, False, -1),
    (torch.bfloat16, 1, 3, 1, True, 100),
    (torch.bfloat16, 2, 3, 1, True, 100),
]


@pytest.mark.parametrize("kv_dtype,topk,steps,page_size,swa,window", ROUNDS)
def test_draft_round(kv_dtype, topk, steps, page_size, swa, window):
    print(f"[case] draft round {kv_dtype} topk={topk} steps={steps} ps={page_size} swa={swa} w={window}",
          flush=True)
    gen = torch.Generator().manual_seed(21 + topk + steps + page_size)
    eng = fakes.Engine(DEV, hq=HQ, hkv=HKV, head_dim=D, kv_dtype=kv_dtype, pool_size=8000, max_reqs=6,
                       context_len=4096, swa=swa)
    eng.runner.page_size = page_size
    layer = _layer(kv_dtype, HQ, HKV, D, window)
    reqs = [4, 1, 3]
    for r, n in zip(reqs, (700, 33, 1500)):
        s = eng.alloc(r, n)
        eng.fill(0, s, _rand(gen, n, HKV, D), _rand(gen, n, HKV, D), layer)
    cont = _container(eng, topk, steps, layer)
    seq, fb = _engine_round(eng, reqs, topk, steps)
    cont.init_forward_metadata(fb)
    r2t = eng.req_to_token.cpu().tolist()
    if topk > 1:
        got = cont.current.table.cpu()
        want = meta.draft_rows(r2t, reqs, seq, topk, steps)
        for r, row in enumerate(want):
            assert got[r, :len(row)].tolist() == row, f"draft table row {r}"
    if swa:
        mapping = eng.pool.full_to_swa_index_mapping.cpu().tolist()
        got = cont.current.swa_table.cpu()
        for r, row in enumerate(meta.draft_rows(r2t, reqs, seq, topk, steps, mapping=mapping)):
            assert got[r, :len(row)].tolist() == row, f"swa draft row {r}"
    for i in range(steps - 1):
        rows, loc = _pass_rows(eng, reqs, seq, topk, steps, i)
        n = len(rows)
        fb.out_cache_loc = torch.tensor(loc, dtype=torch.int64, device=DEV)
        q, k, v = _rand(gen, n, HQ * D), _rand(gen, n, HKV, D), _rand(gen, n, HKV, D)
        out = cont.attn_backends[i].forward_decode(q, k, v, layer, fb)  # writes pass i's K/V first
        torch.cuda.synchronize()
        assert_attn_close(out.reshape(n, HQ, D), _reference(eng, layer, q, rows, swa=swa),
                          what=f"pass {i} topk={topk} ps={page_size} swa={swa}")


@pytest.mark.parametrize("topk", [1, 2])
def test_draft_rounds_in_a_hip_graph(topk):
    """The engine captures a round's passes once and replays them every round: metadata
    planned into fixed buffers outside the graph, passes replayed inside it."""
    print(f"[case] draft rounds in a graph topk={topk}", flush=True)
    steps = 3
    gen = torch.Generator().manual_seed(31 + topk)
    eng = fakes.Engine(DEV, hq=HQ, hkv=HKV, head_dim=D, kv_dtype=torch.bfloat16, pool_size=9000, max_reqs=4,
                       context_len=4096)
    layer = _layer(torch.bfloat16, HQ, HKV, D)
    reqs = [2, 0]
    for r, n in zip(reqs, (300, 1200)):
        s = eng.alloc(r, n)
        eng.fill(0, s, _rand(gen, n, HKV, D), _rand(gen, n, HKV, D), layer)
    cont = _container(eng, topk, steps, layer)
    cont.init_cuda_graph_state(max_bs=4, max_num_tokens=4 * topk)
    n = len(reqs) * topk
    q = [_rand(gen, n, HQ * D) for _ in range(steps - 1)]
    kv = [(_rand(gen, n, HKV, D), _rand(gen, n, HKV, D)) for _ in range(steps - 1)]
    locs = [torch.zeros(n, dtype=torch.int64, device=DEV) for _ in range(steps - 1)]

    def new_round():
        seq, fb = _engine_round(eng, reqs, topk, steps)
        plan_rows = []
        for i in range(steps - 1):
            rows, loc = _pass_rows(eng, reqs, seq, topk, steps, i)
            locs[i].copy_(torch.tensor(loc, dtype=torch.int64))
            q[i].copy_(_rand(gen, n, HQ * D))
            kv[i][0].copy_(_rand(gen, n, HKV, D))
            kv[i][1].copy_(_rand(gen, n, HKV, D))
            plan_rows.append(rows)
        return fb, plan_rows

    def passes():
        outs = []
        for i in range(steps - 1):
            fbi = SimpleNamespace(out_cache_loc=locs[i])
            outs.append(cont.attn_backends[i].forward_decode(q[i], kv[i][0], kv[i][1], layer, fbi))
        return outs

    fb, _ = new_round()
    cont.init_forward_metadata_capture_cuda_graph(fb)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        passes()  # warm-up outside the graph
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = passes()
    for it in range(3):
        fb, plan_rows = new_round()
        cont.init_forward_metadata_replay_cuda_graph(fb, len(reqs))
        graph.replay()
        torch.cuda.synchronize()
        got = [o.clone() for o in outs]
        eager = passes()  # rewrites the same K/V, then attends again
        torch.cuda.synchronize()
        for i in range(steps - 1):
            assert torch.equal(got[i], eager[i]), f"replay {it} pass {i}"
            assert_attn_close(got[i].reshape(n, HQ, D), _reference(eng, layer, q[i], plan_rows[i]),
                              what=f"replay {it} pass {i}")
