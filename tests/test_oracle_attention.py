"""Pins oracle/attention.py (and cross-checks oracle/torch_native.py).

Each check is chosen so that a plausible mistake fails it: a dropped scale, a
wrong GQA mapping (h % Hkv instead of h // G), an off-by-one causal bound, a
transposed operand, a page-table index error.
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attention as A
from oracle import torch_native as TN
from sglang_restomod_amd import workloads


def _rand(*shape, seed=0):
    return np.random.default_rng(seed).standard_normal(shape)


@pytest.mark.parametrize("D", [16, 64, 128, 256])
def test_matches_sdpa_with_causal_prefix_mask(D):
    """Extend vs torch SDPA with an explicit causal-with-prefix mask and GQA repeat
    (the form of the reference's tests/test_attention_v100_gpu.py:28-46), at the
    kernels' head dims too."""
    P, E, H, Hkv = 37, 11, 8, 2
    n = P + E
    q, k, v = _rand(E, H, D, seed=1), _rand(n, Hkv, D, seed=2), _rand(n, Hkv, D, seed=3)
    out = A.extend(q, k, v, np.arange(n)[None, :], [0], [P], [E], softmax_scale=D ** -0.5)
    qq = torch.from_numpy(q).transpose(0, 1)[None]
    kk = torch.from_numpy(k).transpose(0, 1)[None].repeat_interleave(H // Hkv, dim=1)
    vv = torch.from_numpy(v).transpose(0, 1)[None].repeat_interleave(H // Hkv, dim=1)
    mask = (torch.arange(n)[None, :] <= torch.arange(P, n)[:, None])[None, None]
    ref = F.scaled_dot_product_attention(qq, kk, vv, attn_mask=mask, scale=D ** -0.5)[0].transpose(0, 1)
    np.testing.assert_allclose(out, ref.numpy(), atol=1e-12)


def test_brute_force_tiny():
    R, n, D = 3, 5, 4
    q, k, v = _rand(R, D, seed=4), _rand(n, D, seed=5), _rand(n, D, seed=6)
    vis = np.array([[1, 1, 0, 0, 0], [1, 1, 1, 1, 1], [0, 0, 1, 0, 1]], dtype=bool)
    bf = A.brute_force(q, k, v, 0.7, vis)
    lo = np.array([0, 0, 2])
    hi = np.array([2, 5, 5])
    got = A._attend(q, k, v, 0.7, lo, hi)
    # row 2 sees keys 2..4 in the range form but only 2 and 4 in the brute force mask
    np.testing.assert_allclose(got[:2], bf[:2], atol=1e-12)
    vis2 = vis.copy()
    vis2[2] = [0, 0, 1, 1, 1]
    np.testing.assert_allclose(got[2], A.brute_force(q, k, v, 0.7, vis2)[2], atol=1e-12)


def test_one_visible_key_returns_its_value_row():
    H, Hkv, D = 4, 2, 8
    k, v = _rand(3, Hkv, D, seed=7), _rand(3, Hkv, D, seed=8)
    q = _rand(1, H, D, seed=9)
    out = A.decode(q, k, v, np.array([[2, 0, 1]]), [0], [1], softmax_scale=1.0, v_scale=0.5)
    for h in range(H):
        np.testing.assert_allclose(out[0, h], 0.5 * v[2, h // 2], atol=1e-14)


def test_gqa_maps_head_to_h_div_group():
    H, Hkv, D, n = 6, 2, 8, 9
    q, k, v = _rand(1, H, D, seed=10), _rand(n, Hkv, D, seed=11), _rand(n, Hkv, D, seed=12)
    out = A.decode(q, k, v, np.arange(n)[None], [0], [n], softmax_scale=0.3)
    for h in range(H):
        ref = A.brute_force(q[0, h][None], k[:, h // 3], v[:, h // 3], 0.3)[0]
        np.testing.assert_allclose(out[0, h], ref, atol=1e-12)
        wrong = A.brute_force(q[0, h][None], k[:, h % 2], v[:, h % 2], 0.3)[0]
        if h // 3 != h % 2:
            assert not np.allclose(out[0, h], wrong)


def test_equal_scores_average_the_values():
    n, D = 7, 4
    v = _rand(n, 1, D, seed=13)
    k = np.zeros((n, 1, D))
    q = _rand(1, 2, D, seed=14)
    out = A.decode(q, k, v, np.arange(n)[None], [0], [n], softmax_scale=1.0)
    np.testing.assert_allclose(out[0, 0], v[:, 0].mean(axis=0), atol=1e-14)


def test_causal_bound_is_inclusive():
    """Query i of a sequence with prefix P sees key P + i (the diagonal) but not P + i + 1."""
    P, E, D = 2, 3, 4
    n = P + E
    k = np.zeros((n, 1, D))
    v = np.eye(n)[:, None, :D] if n <= D else np.arange(n, dtype=float)[:, None, None].repeat(D, axis=2)
    q = np.zeros((E, 1, D))
    out = A.extend(q, k, v, np.arange(n)[None], [0], [P], [E], softmax_scale=1.0)
    for i in range(E):
        np.testing.assert_allclose(out[i, 0, 0], np.arange(P + i + 1).mean(), atol=1e-14)


def test_permuted_slots_match_the_identity_layout():
    H, Hkv, D, n = 4, 2, 8, 20
    q, k, v = _rand(1, H, D, seed=15), _rand(n, Hkv, D, seed=16), _rand(n, Hkv, D, seed=17)
    base = A.decode(q, k, v, np.arange(n)[None], [0], [n], softmax_scale=0.5)
    perm = np.random.default_rng(3).permutation(n)
    kp, vp = np.empty_like(k), np.empty_like(v)
    kp[perm], vp[perm] = k, v  # logical position j now lives in slot perm[j]
    got = A.decode(q, kp, vp, perm[None], [0], [n], softmax_scale=0.5)
    np.testing.assert_allclose(got, base, atol=1e-12)


def test_page_table_slots():
    t = np.array([[5, 2, 9]])
    assert A.slots_from_page_table(t, 0, 7, 3).tolist() == [15, 16, 17, 6, 7, 8, 27]


def test_window_is_a_left_bound_for_non_causal_rows():
    P, E, D = 4, 3, 2
    n = P + E
    k = np.zeros((n, 1, D))
    v = np.arange(n, dtype=float)[:, None, None].repeat(D, axis=2)
    q = np.zeros((E, 1, D))
    out = A.extend(q, k, v, np.arange(n)[None], [0], [P], [E], softmax_scale=1.0, causal=False, sliding_window=1)
    for i in range(E):
        lo = P + i - 1
        np.testing.assert_allclose(out[i, 0, 0], np.arange(lo, n).mean(), atol=1e-14)


def test_empty_sequence_gives_zero():
    q = _rand(1, 2, 4, seed=18)
    out = A.decode(q, np.zeros((1, 1, 4)), np.ones((1, 1, 4)), np.zeros((1, 1), dtype=int), [0], [0],
                   softmax_scale=1.0)
    assert np.all(out == 0)


def test_scales_fold_into_scores_and_outputs():
    H, Hkv, D, n = 2, 1, 8, 6
    q, k, v = _rand(1, H, D, seed=19), _rand(n, Hkv, D, seed=20), _rand(n, Hkv, D, seed=21)
    a = A.decode(q, k, v, np.arange(n)[None], [0], [n], softmax_scale=0.25, k_scale=2.0, v_scale=3.0)
    b = A.decode(q, 2.0 * k, 3.0 * v, np.arange(n)[None], [0], [n], softmax_scale=0.25)
    np.testing.assert_allclose(a, b, atol=1e-12)


@pytest.mark.parametrize("index", [0, 1, 2, 4])
def test_torch_native_matches_the_float64_oracle(index):
    w = workloads.make(index, batch=3, scale_lens=0.02)
    qf = w.q.double().numpy()
    kf = w.k_pool.double().numpy()
    vf = w.v_pool.double().numpy()
    r2t = w.req_to_token.numpy()
    rpi = w.req_pool_indices.numpy()
    if w.mode == "decode":
        ref = A.decode(qf, kf, vf, r2t, rpi, w.seq_lens.numpy(), softmax_scale=w.softmax_scale)
        got = TN.decode(w.q, w.k_pool, w.v_pool, w.req_to_token, w.req_pool_indices, w.seq_lens,
                        softmax_scale=w.softmax_scale)
    else:
        ref = A.extend(qf, kf, vf, r2t, rpi, w.prefix_lens.numpy(), w.extend_lens.numpy(),
                       softmax_scale=w.softmax_scale)
        got = TN.extend(w.q, w.k_pool, w.v_pool, w.req_to_token, w.req_pool_indices, w.prefix_lens.tolist(),
                        w.extend_lens.tolist(), softmax_scale=w.softmax_scale)
    np.testing.assert_allclose(got.numpy(), ref, atol=2e-5)


def test_torch_native_fp8_dequant_matches():
    w = workloads.make(3, batch=2, scale_lens=0.01, kv_format="e5m2")
    kf = w.k_pool.double().numpy()
    vf = w.v_pool.double().numpy()
    ref = A.decode(w.q.double().numpy(), kf, vf, w.req_to_token.numpy(), w.req_pool_indices.numpy(),
                   w.seq_lens.numpy(), softmax_scale=w.softmax_scale, k_scale=w.k_scale, v_scale=w.v_scale)
    got = TN.decode(w.q, w.k_pool, w.v_pool, w.req_to_token, w.req_pool_indices, w.seq_lens,
                    softmax_scale=w.softmax_scale, k_scale=w.k_scale, v_scale=w.v_scale)
    np.testing.assert_allclose(got.numpy(), ref, atol=2e-5)


def test_workload_totals_match_the_documented_example():
    assert sum(workloads.seq_lengths(1)) == 295239
    assert sum(workloads.seq_lengths(3)) == 2147090
    assert sum(workloads.seq_lengths(4)) == 254648
    g = torch.Generator().manual_seed(2)
    P = torch.randint(0, 4097, (8,), generator=g)
    E = torch.randint(256, 2049, (8,), generator=g)
    assert (int(P.sum()), int(E.sum())) == (12453, 11179)


def test_flop_and_byte_counts_are_closed_form():
    w = workloads.make(2, batch=2, scale_lens=0.01)
    P, E = w.prefix_lens.tolist(), w.extend_lens.tolist()
    pairs = sum(sum(p + i + 1 for i in range(e)) for p, e in zip(P, E))
    assert workloads.algorithmic_flops(w) == 4 * w.dim * w.heads * pairs
    d = workloads.make(0)
    assert workloads.algorithmic_bytes(d) == 2 * 512 * 8 * 128 * 2 + 4 * 512 + 2 * 32 * 128 * 2


@pytest.mark.parametrize("index,fmt", [(0, None), (1, None), (2, None), (4, None), (3, "e4m3"), (3, "e5m2"),
                                       (5, None), (6, None)])
def test_float64_torch_form_matches_the_oracle(index, fmt):
    """oracle.torch_f64 (the full-size reference of the GPU tests) against the numpy oracle
    on every workload's shape, shrunk: identical to float64 rounding."""
    from oracle import torch_f64 as F64

    w = workloads.make(index, batch=3, scale_lens=0.03, kv_format=fmt or "e4m3")
    kf = w.k_pool.double().numpy()
    vf = w.v_pool.double().numpy()
    r2t, rpi = w.req_to_token.numpy(), w.req_pool_indices.numpy()
    common = dict(softmax_scale=w.softmax_scale, k_scale=w.k_scale, v_scale=w.v_scale)
    if w.mode == "decode":
        ref = A.decode(w.q.double().numpy(), kf, vf, r2t, rpi, w.seq_lens.numpy(), **common)
    else:
        ref = A.extend(w.q.double().numpy(), kf, vf, r2t, rpi, w.prefix_lens.numpy(), w.extend_lens.numpy(),
                       **common)
    slots = F64.rows_of_table(w.req_to_token, w.req_pool_indices, w.seq_lens_cpu)
    got = F64.attend(w.q, w.k_pool, w.v_pool, slots, w.query_start_loc.tolist(), w.prefix_lens.tolist(),
                     w.seq_lens_cpu, **common)
    np.testing.assert_allclose(got.numpy(), ref, rtol=0, atol=1e-12)


@pytest.mark.parametrize("window,causal", [(5, True), (0, True), (7, False)])
def test_float64_torch_form_windows_and_masks(window, causal):
    from oracle import torch_f64 as F64

    g = torch.Generator().manual_seed(5)
    q = torch.randn(9, 4, 16, generator=g, dtype=torch.float64)
    k = torch.randn(40, 2, 16, generator=g, dtype=torch.float64)
    v = torch.randn(40, 2, 16, generator=g, dtype=torch.float64)
    slots = [torch.randperm(40, generator=g)[:30], torch.randperm(40, generator=g)[:12]]
    qsl, pre, seq = [0, 6, 9], [24, 9], [30, 12]
    ref = A.paged_attention(q.numpy(), k.numpy(), v.numpy(), [s.numpy() for s in slots], qsl, pre, seq,
                            softmax_scale=0.3, causal=causal, sliding_window=window)
    got = F64.attend(q, k, v, slots, qsl, pre, seq, softmax_scale=0.3, causal=causal, sliding_window=window)
    np.testing.assert_allclose(got.numpy(), ref, rtol=0, atol=1e-12)
