"""GPU parity of the split-KV decode / verify kernels against the float64 oracle.

Inputs follow the seeded workload generator (page size 1, slots scattered over
the whole pool by a global permutation, request rows permuted inside a larger
req_to_token). Small cases check every sequence; full-size workloads check a
sample of sequences (each sequence's output depends only on its own keys).
"""

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


def _decode_case(gpu, index, batch=None, scale_lens=1.0, kv_format="e4m3", check=None, **kw):
    w = workloads.make(index, device=gpu, kv_format=kv_format, batch=batch, scale_lens=scale_lens)
    print(f"[case] decode workload={w.name} batch={w.batch} kv={w.k_pool.dtype} kw={kw}", flush=True)
    ops = _ops()
    out = ops.grouped_decode_forward(
        w.q, w.k_pool, w.v_pool, w.req_to_token, w.seq_lens,
        softmax_scale=w.softmax_scale, k_scale=w.k_scale, v_scale=w.v_scale,
        row_index=w.req_pool_indices, max_seq_len_hint=max(w.seq_lens_cpu), **kw,
    )
    torch.cuda.synchronize()
    rows = list(range(w.batch)) if check is None else check
    _check_decode_rows(w, out, rows, kw.get("sliding_window_size", -1))
    return w, out


def _gather_f64(pool, slots):
    """Rows of a pool as float64 on the CPU (fp8 gathered as bytes, decoded by torch's cast)."""
    if pool.dtype in (torch.float8_e4m3fn, torch.float8_e5m2):
        raw = pool.view(torch.uint8)[slots].cpu()
        return raw.view(pool.dtype).float().numpy().astype(np.float64)
    return pool[slots].float().cpu().numpy().astype(np.float64)


def _check_decode_rows(w, out, rows, window=-1):
    r2t = w.req_to_token.cpu().numpy()
    rpi = w.req_pool_indices.cpu().numpy()
    q = to_f64(w.q)
    for b in rows:
        n = w.seq_lens_cpu[b]
        slots = torch.from_numpy(r2t[rpi[b], :n].astype(np.int64)).to(w.k_pool.device)
        kb, vb = _gather_f64(w.k_pool, slots), _gather_f64(w.v_pool, slots)
        # pools of just this sequence's keys, slots 0..n-1
        table = np.arange(max(n, 1), dtype=np.int64)[None, :]
        ref = oracle.decode(q[b:b + 1], kb, vb, table, [0], [n], softmax_scale=w.softmax_scale,
                            k_scale=w.k_scale, v_scale=w.v_scale, sliding_window=window)
        assert_attn_close(out[b:b + 1], ref, what=f"{w.name} seq {b} (ctx {n})")


def test_decode_single_sequence_fp16(gpu):
    """B=1, ctx 512, 32/8 heads, fp16: the CPU-runnable reference case, every output."""
    _decode_case(gpu, 0)


def test_decode_batched_bf16_small(gpu):
    _decode_case(gpu, 1, batch=8, scale_lens=0.125)


def test_decode_batched_bf16_full_sample(gpu):
    """The full 64-sequence ragged workload; shortest, longest and a spread checked."""
    order = np.argsort(workloads.seq_lengths(1))
    check = sorted({int(order[0]), int(order[-1]), 3, 17, 40, 63})
    _decode_case(gpu, 1, check=check)


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
def test_decode_fp8_small(gpu, fmt):
    _decode_case(gpu, 3, batch=6, scale_lens=0.05, kv_format=fmt)


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
def test_decode_fp8_full_sample(gpu, fmt):
    _decode_case(gpu, 3, kv_format=fmt, check=[0, 77, 127])


def test_decode_grid_size_does_not_change_the_result(gpu):
    """Different persistent grids cut the tile list differently (segments shared by 1..many
    waves, waves with empty ranges); the merged result must not depend on it."""
    w = workloads.make(1, device=gpu, batch=4, scale_lens=0.25)
    ops = _ops()
    outs = []
    for nwg in (1, 3, 37, 256, 1000):
        outs.append(ops.grouped_decode_forward(
            w.q, w.k_pool, w.v_pool, w.req_to_token, w.seq_lens, softmax_scale=w.softmax_scale,
            row_index=w.req_pool_indices, num_workgroups=nwg).float())
    torch.cuda.synchronize()
    _check_decode_rows(w, outs[0].to(w.q.dtype), range(w.batch))
    for o in outs[1:]:
        torch.testing.assert_close(o, outs[0], atol=2e-3, rtol=0)


def _synthetic(gpu, lengths, heads, heads_kv, dim=128, dtype=torch.bfloat16, seed=0, page_size=1):
    """Random pool + a reversed-page table so that a page-table mistake cannot pass."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    B = len(lengths)
    pages_per = [max(1, math.ceil(n / page_size)) for n in lengths]
    total_pages = sum(pages_per) + 1
    k = torch.randn(total_pages * page_size, heads_kv, dim, generator=g).to(dtype).to(gpu)
    v = torch.randn(total_pages * page_size, heads_kv, dim, generator=g).to(dtype).to(gpu)
    q = torch.randn(B, heads, dim, generator=g).to(dtype).to(gpu)
    width = max(pages_per)
    table = torch.zeros(B, width, dtype=torch.int32)
    nxt = 1
    for b, cnt in enumerate(pages_per):
        table[b, :cnt] = torch.arange(nxt, nxt + cnt, dtype=torch.int32).flip(0)
        nxt += cnt
    return q, k, v, table.to(gpu), torch.tensor(lengths, dtype=torch.int32, device=gpu)


def _check_table_decode(q, k, v, table, seq, page_size, out, scale, window=-1):
    qs = to_f64(q)
    kf, vf = to_f64(k), to_f64(v)
    t = table.cpu().numpy()
    for b, n in enumerate(seq.cpu().tolist()):
        slots = oracle.slots_from_page_table(t, b, n, page_size)
        ref = oracle.paged_attention(qs[b:b + 1], kf, vf, [slots], [0, 1], [max(n - 1, 0)], [n],
                                     softmax_scale=scale, sliding_window=window)
        assert_attn_close(out[b:b + 1], ref, what=f"seq {b} ctx {n}")


@pytest.mark.parametrize("heads,heads_kv", [(8, 8), (32, 8), (40, 8), (64, 4), (128, 2)])
def test_decode_gqa_ratios(gpu, heads, heads_kv):
    lengths = [1, 31, 32, 33, 300, 1000]
    q, k, v, table, seq = _synthetic(gpu, lengths, heads, heads_kv)
    out = _ops().grouped_decode_forward(q, k, v, table, seq, softmax_scale=128 ** -0.5, max_seq_len_hint=1000)
    torch.cuda.synchronize()
    _check_table_decode(q, k, v, table, seq, 1, out, 128 ** -0.5)


@pytest.mark.parametrize("heads,heads_kv,dim", [(64, 4, 128), (12, 2, 256), (48, 2, 64)])
def test_decode_persistent_merge_of_several_row_sets(gpu, heads, heads_kv, dim):
    """The persistent split-KV path (no length hint) over sequences long enough that many
    waves share each segment, at GQA groups whose rows fill more than one merge row set
    (16 rows at D=128 and 6 at D=256: one merge workgroup per row set; 24 at D=64)."""
    lengths = [5000, 7000, 300, 1]
    q, k, v, table, seq = _synthetic(gpu, lengths, heads, heads_kv, dim=dim)
    out = _ops().grouped_decode_forward(q, k, v, table, seq, softmax_scale=dim ** -0.5)
    torch.cuda.synchronize()
    _check_table_decode(q, k, v, table, seq, 1, out, dim ** -0.5)


def test_decode_page_size_16_table(gpu):
    """The reference kernels' paged layout: [pages, 16, Hkv, D] through a page table."""
    lengths = [37, 53, 67, 200]
    q, k, v, table, seq = _synthetic(gpu, lengths, 32, 8, dtype=torch.float16, page_size=16)
    k4 = k.view(-1, 16, 8, 128)
    v4 = v.view(-1, 16, 8, 128)
    out = _ops().grouped_decode_forward(q, k4, v4, table, seq, softmax_scale=0.1)
    torch.cuda.synchronize()
    _check_table_decode(q, k, v, table, seq, 16, out, 0.1)


@pytest.mark.parametrize("dim,dtype", [(96, torch.bfloat16), (512, torch.float16)])
def test_decode_page_size_16_table_other_head_dims(gpu, dim, dtype):
    """The 16-token page layout through the any-head-dim kernel's decode."""
    lengths = [1, 37, 53, 200]
    q, k, v, table, seq = _synthetic(gpu, lengths, 16, 4, dim=dim, dtype=dtype, page_size=16)
    k4 = k.view(-1, 16, 4, dim)
    v4 = v.view(-1, 16, 4, dim)
    out = _ops().grouped_decode_forward(q, k4, v4, table, seq, softmax_scale=dim ** -0.5)
    torch.cuda.synchronize()
    _check_table_decode(q, k, v, table, seq, 16, out, dim ** -0.5)


def test_decode_zero_length_gives_zero(gpu):
    q, k, v, table, seq = _synthetic(gpu, [0, 5], 32, 8)
    out = _ops().grouped_decode_forward(q, k, v, table, seq, softmax_scale=0.1)
    torch.cuda.synchronize()
    assert torch.count_nonzero(out[0]) == 0
    _check_table_decode(q[1:], k, v, table[1:], seq[1:], 1, out[1:], 0.1)


def test_decode_sliding_window(gpu):
    lengths = [10, 100, 1000, 3000]
    q, k, v, table, seq = _synthetic(gpu, lengths, 32, 8)
    out = _ops().grouped_decode_forward(q, k, v, table, seq, softmax_scale=0.1, sliding_window_size=64,
                                        max_seq_len_hint=3000)
    torch.cuda.synchronize()
    _check_table_decode(q, k, v, table, seq, 1, out, 0.1, window=64)


def test_decode_one_visible_key_returns_that_value_row(gpu):
    q, k, v, table, seq = _synthetic(gpu, [1, 1, 1], 16, 2)
    out = _ops().grouped_decode_forward(q, k, v, table, seq, softmax_scale=0.3)
    torch.cuda.synchronize()
    for b in range(3):
        slot = int(table[b, 0])
        want = v[slot].repeat_interleave(8, dim=0)
        torch.testing.assert_close(out[b], want, atol=0, rtol=0)


# ---------------------------------------------------------------------------
# verify
# ---------------------------------------------------------------------------

def _verify_case(gpu, batch=None, scale_lens=1.0, check=None, draft=None):
    w = workloads.make(4, device=gpu, batch=batch, scale_lens=scale_lens)
    print(f"[case] verify workload={w.name} batch={w.batch}", flush=True)
    ops = _ops()
    T = int(w.extend_lens[0])
    out = ops.paged_verify_forward(
        w.q, w.k_pool, w.v_pool, w.req_to_token, w.seq_lens, w.query_start_loc, w.prefix_lens,
        max_q_per_seq=T, softmax_scale=w.softmax_scale, row_index=w.req_pool_indices,
        max_seq_len_hint=max(w.seq_lens_cpu),
    )
    torch.cuda.synchronize()
    r2t = w.req_to_token.cpu().numpy()
    rpi = w.req_pool_indices.cpu().numpy()
    q = to_f64(w.q)
    rows = range(w.batch) if check is None else check
    for b in rows:
        n = w.seq_lens_cpu[b]
        P = n - T
        slots = torch.from_numpy(r2t[rpi[b], :n].astype(np.int64)).to(gpu)
        kb, vb = _gather_f64(w.k_pool, slots), _gather_f64(w.v_pool, slots)
        ref = oracle.verify(q[b * T:(b + 1) * T], kb, vb, np.arange(n)[None, :], [0], [P], T,
                            softmax_scale=w.softmax_scale)
        assert_attn_close(out[b * T:(b + 1) * T], ref, what=f"verify seq {b} (prefix {P})")


def test_verify_small(gpu):
    _verify_case(gpu, batch=6, scale_lens=0.05)


def test_verify_full_sample(gpu):
    _verify_case(gpu, check=[0, 13, 31])


def test_verify_ragged_query_counts(gpu):
    """Sequences with 1..7 draft rows in one batch, 32/8 heads (rows per kv head up to 28)."""
    g = torch.Generator().manual_seed(5)
    B, H, Hkv, D = 5, 32, 8, 128
    qlens = [1, 3, 7, 4, 2]
    prefix = [0, 17, 250, 1000, 64]
    seq = [p + e for p, e in zip(prefix, qlens)]
    pool = sum(seq) + 1
    k = torch.randn(pool, Hkv, D, generator=g).to(torch.bfloat16).to(gpu)
    v = torch.randn(pool, Hkv, D, generator=g).to(torch.bfloat16).to(gpu)
    T = sum(qlens)
    q = torch.randn(T, H, D, generator=g).to(torch.bfloat16).to(gpu)
    perm = torch.randperm(pool - 1, generator=g) + 1
    table = torch.zeros(B, max(seq), dtype=torch.int32)
    off = 0
    for b, n in enumerate(seq):
        table[b, :n] = perm[off:off + n].to(torch.int32)
        off += n
    qsl = torch.tensor([0] + list(np.cumsum(qlens)), dtype=torch.int32)
    out = _ops().paged_verify_forward(
        q, k, v, table.to(gpu), torch.tensor(seq, dtype=torch.int32, device=gpu), qsl.to(gpu),
        torch.tensor(prefix, dtype=torch.int32, device=gpu), max_q_per_seq=max(qlens),
        softmax_scale=D ** -0.5)
    torch.cuda.synchronize()
    ref = oracle.paged_attention(to_f64(q), to_f64(k), to_f64(v), [table[b].numpy() for b in range(B)],
                                 qsl.tolist(), prefix, seq, softmax_scale=D ** -0.5)
    assert_attn_close(out, ref, what="ragged verify")


@pytest.mark.parametrize("mode", ["decode", "decode_pieces", "verify"])
def test_poisoned_workspace_and_output(gpu, mode):
    """The workspace needs no initialisation: filled with 0xFF bytes (NaN pieces, -1
    descriptors) and reused by a smaller call, and with the output pre-filled with NaN,
    every result is the one a fresh workspace gives, bit for bit. decode_pieces: the small
    decode split over key pieces (a length bound given), whose pieces live there too."""
    ops = _ops()
    idx = 4 if mode == "verify" else 1
    big = workloads.make(idx, device=gpu, batch=12 if mode != "decode_pieces" else 2, scale_lens=0.3)
    small = workloads.make(idx, device=gpu, batch=3 if mode != "decode_pieces" else 1, scale_lens=0.05)

    def run(w, ws, out):
        if mode.startswith("decode"):
            hint = max(w.seq_lens_cpu) if mode == "decode_pieces" else None
            if hint is not None:
                assert ops.decode_kernel(w.batch, w.heads, w.heads_kv, w.dim, hint) == "any_kernel"
            return ops.grouped_decode_forward(
                w.q, w.k_pool, w.v_pool, w.req_to_token, w.seq_lens, softmax_scale=w.softmax_scale,
                row_index=w.req_pool_indices, out=out, workspace=ws, max_seq_len_hint=hint)
        T = int(w.extend_lens[0])
        return ops.paged_verify_forward(
            w.q, w.k_pool, w.v_pool, w.req_to_token, w.seq_lens, w.query_start_loc, w.prefix_lens,
            max_q_per_seq=T, softmax_scale=w.softmax_scale, out=out, row_index=w.req_pool_indices,
            workspace=ws)

    fresh = ops.splitkv_workspace(torch.device(gpu))
    want = [run(w, fresh, None).clone() for w in (big, small)]
    poisoned = ops.splitkv_workspace(torch.device(gpu))
    poisoned.fill_(0xFF)
    for w, ref in zip((big, small), want):   # the small call sees the big call's leftovers
        out = torch.full_like(ref, float("nan"))
        run(w, poisoned, out)
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"{mode}: a poisoned or stale workspace changed the result"


def test_two_streams_with_their_own_workspaces(gpu):
    """Calls that overlap in time on two streams, each with the shared workspace of its
    own stream, give the results of the same calls run one after another."""
    ops = _ops()
    w1 = workloads.make(1, device=gpu, batch=16, scale_lens=0.4)
    w2 = workloads.make(4, device=gpu, batch=8, scale_lens=0.3)

    def dec(out=None):
        return ops.grouped_decode_forward(w1.q, w1.k_pool, w1.v_pool, w1.req_to_token, w1.seq_lens,
                                          softmax_scale=w1.softmax_scale, row_index=w1.req_pool_indices, out=out)

    def ver(out=None):
        return ops.paged_verify_forward(w2.q, w2.k_pool, w2.v_pool, w2.req_to_token, w2.seq_lens,
                                        w2.query_start_loc, w2.prefix_lens, max_q_per_seq=4,
                                        softmax_scale=w2.softmax_scale, row_index=w2.req_pool_indices, out=out)

    want1, want2 = dec().clone(), ver().clone()
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    o1, o2 = torch.empty_like(want1), torch.empty_like(want2)
    s1.wait_stream(torch.cuda.current_stream())
    s2.wait_stream(torch.cuda.current_stream())
    for _ in range(5):
        with torch.cuda.stream(s1):
            dec(o1)
        with torch.cuda.stream(s2):
            ver(o2)
    torch.cuda.synchronize()
    assert torch.equal(o1, want1) and torch.equal(o2, want2)
