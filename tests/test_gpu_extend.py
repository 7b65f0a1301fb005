"""GPU parity of the MFMA extend kernel against the float64 oracle."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import attention as oracle
from sglang_restomod_amd import workloads
from tests.helpers import assert_attn_close, to_f64

pytestmark = pytest.mark.gpu


def _ops():
    from sglang_restomod_amd.attention.mi355x import ops

    return ops


def _gather_f64(pool, slots):
    if pool.dtype in (torch.float8_e4m3fn, torch.float8_e5m2):
        return pool.view(torch.uint8)[slots].cpu().view(pool.dtype).float().numpy().astype(np.float64)
    return pool[slots].float().cpu().numpy().astype(np.float64)


def _check_rows(q, k_pool, v_pool, slots_of, prefix, qsl, out, rows_of, scale, k_scale=1.0, v_scale=1.0,
                causal=True, window=-1, what=""):
    """Check the listed query rows of each sequence; rows become one-row problems for the oracle."""
    qf = to_f64(q)
    for b, rows in rows_of.items():
        if not rows:
            continue
        n_total = int(prefix[b]) + (int(qsl[b + 1]) - int(qsl[b]))
        slots = torch.as_tensor(slots_of(b, n_total), dtype=torch.int64, device=k_pool.device)
        kb, vb = _gather_f64(k_pool, slots), _gather_f64(v_pool, slots)
        ident = np.arange(n_total)
        got_rows = [int(qsl[b]) + i for i in rows]
        ref = oracle.paged_attention(
            qf[got_rows], kb, vb, [ident] * len(rows), list(range(len(rows) + 1)),
            [int(prefix[b]) + i for i in rows], [n_total] * len(rows),
            softmax_scale=scale, k_scale=k_scale, v_scale=v_scale, causal=causal, sliding_window=window)
        assert_attn_close(out[got_rows], ref, what=f"{what} seq {b} rows {rows[:3]}..")


def _workload_extend(gpu, batch=None, scale_lens=1.0, sample=None, kv_format=None):
    w = workloads.make(2, device=gpu, batch=batch, scale_lens=scale_lens)
    if kv_format is not None:
        from sglang_restomod_amd.workloads import FP8

        w.k_scale, w.v_scale = 0.75, 1.5
        w.k_pool = (w.k_pool.float() / w.k_scale).to(FP8[kv_format])
        w.v_pool = (w.v_pool.float() / w.v_scale).to(FP8[kv_format])
    print(f"[case] extend {w.name} batch={w.batch} kv={w.k_pool.dtype}", flush=True)
    qsl = w.query_start_loc
    E = w.extend_lens.tolist()
    out, _ = _ops().paged_forward(
        w.q, w.k_pool, w.v_pool, w.req_to_token, w.seq_lens, qsl, w.prefix_lens, block_size=1,
        softmax_scale=w.softmax_scale, k_scale=w.k_scale, v_scale=w.v_scale, causal=True,
        row_index=w.req_pool_indices, max_seq_len_hint=max(w.seq_lens_cpu), max_q_len_hint=max(E))
    torch.cuda.synchronize()
    r2t = w.req_to_token.cpu().numpy()
    rpi = w.req_pool_indices.cpu().numpy()
    rows_of = {}
    for b in range(w.batch):
        if sample is None:
            rows_of[b] = list(range(E[b]))
        else:
            rows_of[b] = sorted(set([0, 1, E[b] - 1] + list(range(0, E[b], max(1, E[b] // sample)))))
    _check_rows(w.q, w.k_pool, w.v_pool, lambda b, n: r2t[rpi[b], :n], w.prefix_lens.tolist(),
                qsl.tolist(), out, rows_of, w.softmax_scale, w.k_scale, w.v_scale, what=w.name)


def test_extend_workload_small(gpu):
    _workload_extend(gpu, batch=3, scale_lens=0.1)


def test_extend_workload_full_sampled_rows(gpu):
    _workload_extend(gpu, sample=12)


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
def test_extend_fp8_kv(gpu, fmt):
    _workload_extend(gpu, batch=2, scale_lens=0.08, kv_format=fmt)


def _synthetic(gpu, prefix, extend, heads, heads_kv, dtype=torch.bfloat16, page_size=1, seed=0, dim=128):
    g = torch.Generator().manual_seed(seed)
    B = len(prefix)
    seq = [p + e for p, e in zip(prefix, extend)]
    pages_per = [max(1, math.ceil(n / page_size)) for n in seq]
    total_pages = sum(pages_per) + 1
    k = torch.randn(total_pages * page_size, heads_kv, dim, generator=g).to(dtype).to(gpu)
    v = torch.randn(total_pages * page_size, heads_kv, dim, generator=g).to(dtype).to(gpu)
    T = sum(extend)
    q = torch.randn(T, heads, dim, generator=g).to(dtype).to(gpu)
    perm = (torch.randperm(total_pages - 1, generator=g) + 1).to(torch.int32)
    table = torch.zeros(B, max(pages_per), dtype=torch.int32)
    off = 0
    for b, cnt in enumerate(pages_per):
        table[b, :cnt] = perm[off:off + cnt]
        off += cnt
    qsl = [0]
    for e in extend:
        qsl.append(qsl[-1] + e)
    return q, k, v, table, seq, qsl


def _run_synthetic(gpu, prefix, extend, heads, heads_kv, causal=True, window=-1, dtype=torch.bfloat16,
                   page_size=1, scale=None, dim=128):
    q, k, v, table, seq, qsl = _synthetic(gpu, prefix, extend, heads, heads_kv, dtype, page_size, dim=dim)
    scale = scale or dim ** -0.5
    kc, vc = k, v
    if page_size > 1:
        kc = k.view(-1, page_size, heads_kv, dim)
        vc = v.view(-1, page_size, heads_kv, dim)
    out, _ = _ops().paged_forward(
        q, kc, vc, table.to(gpu), torch.tensor(seq, dtype=torch.int32, device=gpu),
        torch.tensor(qsl, dtype=torch.int32, device=gpu), torch.tensor(prefix, dtype=torch.int32, device=gpu),
        softmax_scale=scale, causal=causal, sliding_window_size=window, block_size=page_size,
        max_q_len_hint=max(extend))
    torch.cuda.synchronize()
    t = table.numpy()
    rows_of = {b: list(range(extend[b])) for b in range(len(prefix))}
    _check_rows(q, k, v, lambda b, n: oracle.slots_from_page_table(t, b, n, page_size), prefix, qsl, out,
                rows_of, scale, causal=causal, window=window, what=f"H{heads}/{heads_kv}")


@pytest.mark.parametrize("heads,heads_kv", [(8, 8), (32, 8), (40, 8), (64, 8), (16, 1)])
def test_extend_gqa_ratios(gpu, heads, heads_kv):
    _run_synthetic(gpu, [0, 64, 300, 7], [48, 32, 129, 200], heads, heads_kv)


def test_extend_without_prefix_and_single_tokens(gpu):
    _run_synthetic(gpu, [0, 0, 5, 1000], [1, 2, 1, 3], 40, 8)


def test_extend_non_causal(gpu):
    _run_synthetic(gpu, [10, 100], [70, 33], 32, 8, causal=False)


def test_extend_sliding_window_causal(gpu):
    _run_synthetic(gpu, [0, 500], [300, 100], 32, 8, window=77)


def test_extend_sliding_window_non_causal(gpu):
    _run_synthetic(gpu, [20, 300], [40, 65], 32, 8, causal=False, window=33)


def test_extend_fp16(gpu):
    _run_synthetic(gpu, [64, 0], [32, 48], 32, 8, dtype=torch.float16)


def test_extend_page_size_16_table(gpu):
    """Reference layout [pages, 16, Hkv, D] with scattered pages (tests/test_attention_v100_gpu.py shapes)."""
    _run_synthetic(gpu, [64, 0], [32, 48], 8, 2, dtype=torch.float16, page_size=16)


@pytest.mark.parametrize("prefix,extend", [(64, 32), (0, 48)])
def test_extend_reference_gpu_test_shape(gpu, prefix, extend):
    """The reference's own extend GPU test at its exact shape: H4 / Hkv2, D=256, fp16,
    16-token pages, prefix 64 + 32 and 0 + 48 new tokens
    (tests/test_attention_v100_gpu.py:49-95). Its pages are in order; here they are
    scattered."""
    _run_synthetic(gpu, [prefix], [extend], 4, 2, dtype=torch.float16, page_size=16, dim=256)


@pytest.mark.parametrize("dim,dtype", [(96, torch.bfloat16), (512, torch.float16)])
def test_extend_page_size_16_table_other_head_dims(gpu, dim, dtype):
    """The 16-token page layout through the any-head-dim kernel's extend (scattered pages,
    prefixes that end inside a page)."""
    _run_synthetic(gpu, [37, 0, 130], [45, 70, 19], 16, 4, dtype=dtype, page_size=16, dim=dim)


def test_extend_ragged_batch_with_empty_sequences(gpu):
    # sequences without new tokens list no row tile; the others must still be served
    _run_synthetic(gpu, [30, 0, 400, 9, 0], [0, 70, 0, 300, 1], 40, 8)


def test_extend_more_sequences_than_one_scan_pass(gpu):
    """1,100 sequences: the work list's prefix sum over sequences runs in two passes."""
    g = torch.Generator().manual_seed(5)
    B = 1100
    extend = torch.randint(0, 4, (B,), generator=g).tolist()
    prefix = torch.randint(0, 90, (B,), generator=g).tolist()
    _run_synthetic(gpu, prefix, extend, 16, 8)


def test_extend_work_list_lists_every_row_tile_heaviest_first(gpu):
    prefix, extend, heads, heads_kv = [0, 3000, 17, 800, 0], [700, 40, 0, 1500, 5], 40, 8
    q, k, v, table, seq, qsl = _synthetic(gpu, prefix, extend, heads, heads_kv)
    ops = _ops()
    B, T, G = len(prefix), q.shape[0], heads // heads_kv
    ws = ops.extend_workspace(q.device, T, heads, heads_kv, B)
    ws.fill_(0x5A)
    ops.paged_extend_forward(
        q, k, v, table.to(gpu), torch.tensor(seq, dtype=torch.int32, device=gpu),
        torch.tensor(qsl, dtype=torch.int32, device=gpu), torch.tensor(prefix, dtype=torch.int32, device=gpu),
        softmax_scale=128 ** -0.5, workspace=ws)
    torch.cuda.synchronize()
    cap = (T * G + 255) // 256 + B
    items = ws[: cap * 8].view(torch.int64).cpu().tolist()
    listed = [(it & 0xFFFFFFFF, it >> 32) for it in items if it != -1]
    assert all(it == -1 for it in items[len(listed):]), "padding must follow the listed tiles"
    want = sorted((b, rt) for b in range(B) for rt in range((extend[b] * G + 255) // 256))
    assert sorted(listed) == want

    def key_tiles(b, rt):  # keys of the tile's last row: causal, no window
        t_last = min(extend[b] - 1, (rt * 256 + 255) // G)
        return (min(seq[b], prefix[b] + t_last + 1) + 63) // 64

    costs = [key_tiles(b, rt) for b, rt in listed]
    assert costs == sorted(costs, reverse=True)


def test_extend_in_a_hip_graph_replays_new_splits():
    """A captured extend (fixed token count and batch) replays correctly when the split of
    the tokens across sequences and the prefixes change: the work list is rebuilt on the
    device at every replay."""
    heads, heads_kv, T = 40, 8, 300
    splits = [([10, 0, 77], [100, 150, 50]), ([400, 5, 0], [1, 298, 1]), ([0, 0, 0], [300, 0, 0])]
    prefix0, extend0 = splits[0]
    # one pool large enough for every split
    gpu_dev = torch.device("cuda:0")
    q, k, v, table, _, _ = _synthetic(gpu_dev, [700, 700, 700], [300, 300, 300],
                                      heads, heads_kv)
    ops = _ops()
    B = 3
    qs = torch.randn(T, heads, 128, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16).to(gpu_dev)
    seq_b = torch.zeros(B, dtype=torch.int32, device=gpu_dev)
    qsl_b = torch.zeros(B + 1, dtype=torch.int32, device=gpu_dev)
    pre_b = torch.zeros(B, dtype=torch.int32, device=gpu_dev)
    ws = ops.extend_workspace(gpu_dev, T, heads, heads_kv, B)
    out = torch.empty_like(qs)
    tab = table.to(gpu_dev)

    def load(prefix, extend):
        seq_b.copy_(torch.tensor([p + e for p, e in zip(prefix, extend)], dtype=torch.int32))
        qsl_b.copy_(torch.tensor([0, extend[0], extend[0] + extend[1], sum(extend)], dtype=torch.int32))
        pre_b.copy_(torch.tensor(prefix, dtype=torch.int32))

    def run():
        ops.paged_extend_forward(qs, k, v, tab, seq_b, qsl_b, pre_b, softmax_scale=128 ** -0.5, out=out,
                                 workspace=ws)

    load(prefix0, extend0)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run()
    t = table.numpy()
    for it, (prefix, extend) in enumerate(splits * 2):
        load(prefix, extend)
        graph.replay()
        torch.cuda.synchronize()
        got = out.clone()
        run()
        torch.cuda.synchronize()
        assert torch.equal(got, out), f"replay {it} differs from the eager call"
        qsl = [0, extend[0], extend[0] + extend[1], sum(extend)]
        rows_of = {b: list(range(extend[b])) for b in range(B)}
        _check_rows(qs, k, v, lambda b, n: oracle.slots_from_page_table(t, b, n, 1), prefix, qsl, got,
                    rows_of, 128 ** -0.5, what=f"replay {it}")


def test_paged_forward_with_the_reference_call_shape(gpu):
    """The reference's callers pass the seven tensors positionally, rely on block_size=16
    with a [pages, 16, Hkv, D] cache, and unpack (out, softmax_lse)
    (_paged_adapter.py:567-586, :756-759)."""
    prefix, extend, heads, heads_kv = [40, 0, 200], [30, 17, 64], 16, 4
    q, k, v, table, seq, qsl = _synthetic(gpu, prefix, extend, heads, heads_kv, page_size=16)
    kc, vc = k.view(-1, 16, heads_kv, 128), v.view(-1, 16, heads_kv, 128)
    print("[case] paged_forward reference call shape", flush=True)
    out, lse = _ops().paged_forward(
        q, kc, vc, table.to(gpu), torch.tensor(seq, dtype=torch.int32, device=gpu),
        torch.tensor(qsl, dtype=torch.int32, device=gpu), torch.tensor(prefix, dtype=torch.int32, device=gpu))
    torch.cuda.synchronize()
    assert out.shape == q.shape and out.dtype == q.dtype
    assert lse.shape == (heads, sum(extend)) and lse.dtype == torch.float32
    t = table.numpy()
    rows_of = {b: list(range(extend[b])) for b in range(len(prefix))}
    _check_rows(q, k, v, lambda b, n: oracle.slots_from_page_table(t, b, n, 16), prefix, qsl, out, rows_of,
                128 ** -0.5, what="reference call shape")
    # the same batch as a linear verify (few rows per sequence) also returns the pair
    out2, lse2 = _ops().paged_forward(
        q, kc, vc, table.to(gpu), torch.tensor(seq, dtype=torch.int32, device=gpu),
        torch.tensor(qsl, dtype=torch.int32, device=gpu), torch.tensor(prefix, dtype=torch.int32, device=gpu),
        linear_verify=True)
    torch.cuda.synchronize()
    assert lse2.shape == lse.shape
    _check_rows(q, k, v, lambda b, n: oracle.slots_from_page_table(t, b, n, 16), prefix, qsl, out2, rows_of,
                128 ** -0.5, what="reference call shape, verify route")


def test_bf16_v_outside_fp16_range():
    """Extend runs PV in fp16: bf16 V is converted by round-toward-zero, which clamps values
    beyond fp16's range to +-65504 (and keeps the rest exact, small values included).
    The split-KV decode keeps bf16 V as it is. Both behaviours against the float64 oracle,
    with errors relative to the largest |V| (P is normalised, so O is a convex mix of V)."""
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(77)
    B, hkv, G, D = 2, 2, 2, 128
    prefix, ext = [40, 130], [24, 9]
    seq = [p + e for p, e in zip(prefix, ext)]
    pool = sum(seq) + 1
    k = torch.randn(pool, hkv, D, generator=g).to(torch.bfloat16)
    vf = torch.randn(pool, hkv, D, generator=g)
    pick = torch.rand(pool, hkv, D, generator=g)
    vf = torch.where(pick < 0.03, torch.sign(vf) * 1.0e5, vf)          # beyond fp16's range
    vf = torch.where((pick >= 0.03) & (pick < 0.06), vf * 2.0e4, vf)     # large, inside it
    vf = torch.where((pick >= 0.06) & (pick < 0.09), vf * 1.0e-6, vf)    # below fp16's normal range
    v = vf.to(torch.bfloat16)
    T = sum(ext)
    q = torch.randn(T, hkv * G, D, generator=g).to(torch.bfloat16)
    r2t = torch.zeros(B, max(seq), dtype=torch.int32)
    off = 1
    for b, n in enumerate(seq):
        r2t[b, :n] = torch.arange(off, off + n, dtype=torch.int32)
        off += n
    qsl = [0, ext[0], ext[0] + ext[1]]
    scale = D ** -0.5
    slots = [r2t[b, :n].numpy().astype(np.int64) for b, n in enumerate(seq)]
    kf = k.float().numpy().astype(np.float64)
    v64 = v.float().numpy().astype(np.float64)
    v_clamped = np.clip(v64, -65504.0, 65504.0)
    ref_clamped = oracle.paged_attention(to_f64(q), kf, v_clamped, slots, qsl, prefix, seq, softmax_scale=scale)
    ref_exact = oracle.paged_attention(to_f64(q), kf, v64, slots, qsl, prefix, seq, softmax_scale=scale)
    vmax = float(np.abs(v64).max())
    out = torch.empty(T, hkv * G, D, dtype=torch.float32, device=dev)
    _ops().paged_extend_forward(q.to(dev), k.to(dev), v.to(dev), r2t.to(dev),
                                torch.tensor(seq, dtype=torch.int32, device=dev),
                                torch.tensor(qsl, dtype=torch.int32, device=dev),
                                torch.tensor(prefix, dtype=torch.int32, device=dev), softmax_scale=scale, out=out)
    torch.cuda.synchronize()
    got = out.double().cpu().numpy()
    err_clamped = float(np.abs(got - ref_clamped).max())
    err_exact = float(np.abs(got - ref_exact).max())
    print(f"[result] extend: max |err| vs clamped V {err_clamped:.3e}, vs exact V {err_exact:.3e} (max |V| {vmax:.3e})",
          flush=True)
    assert err_clamped <= 2e-3 * 65504.0, err_clamped
    assert err_exact > 10 * err_clamped  # the clamp is what the kernel computes
    # decode of each sequence's last token: bf16 V used as it is
    qd = torch.stack([q[qsl[b + 1] - 1] for b in range(B)])
    dec = torch.empty(B, hkv * G, D, dtype=torch.float32, device=dev)
    _ops().grouped_decode_forward(qd.to(dev), k.to(dev), v.to(dev), r2t.to(dev),
                                  torch.tensor(seq, dtype=torch.int32, device=dev), softmax_scale=scale, out=dec)
    torch.cuda.synchronize()
    ref_dec = np.stack([ref_exact[qsl[b + 1] - 1] for b in range(B)])
    err_dec = float(np.abs(dec.double().cpu().numpy() - ref_dec).max())
    print(f"[result] decode: max |err| vs exact V {err_dec:.3e}", flush=True)
    assert err_dec <= 2e-3 * vmax, err_dec


@pytest.mark.parametrize("index,dtype", [(6, torch.float16), (6, torch.bfloat16), (2, torch.float16),
                                         (10, torch.float16), (9, torch.bfloat16)])
def test_extend_is_deterministic(index, dtype):
    """Repeated calls on the same inputs give the same bits, fp32 output included: the
    extend batch at head dims 256 (fp16 and bf16), 128, and 192 and 96 (padded onto the
    256 and 128 kernels). A VALU read of an MFMA result before the result is written
    (a hazard the hardware does not interlock) shows up here as run-to-run differences."""
    from sglang_restomod_amd.attention.mi355x import ops

    dev = torch.device("cuda:0")
    w = workloads.make(index, device=dev, batch=4, scale_lens=0.5)
    w.q, w.k_pool, w.v_pool = w.q.to(dtype), w.k_pool.to(dtype), w.v_pool.to(dtype)
    print(f"[case] extend determinism {w.name} {dtype}", flush=True)

    def run(out_dtype):
        out = torch.empty(w.q.shape, dtype=out_dtype, device=dev)
        ops.paged_extend_forward(w.q, w.k_pool, w.v_pool, w.req_to_token, w.seq_lens, w.query_start_loc,
                                 w.prefix_lens, softmax_scale=w.softmax_scale, out=out,
                                 row_index=w.req_pool_indices)
        torch.cuda.synchronize()
        return out

    for out_dtype in (dtype, torch.float32):
        first = run(out_dtype)
        for _ in range(4):
            assert torch.equal(run(out_dtype), first), f"{w.name} {dtype} -> {out_dtype}: run-to-run difference"
