"""A seeded sweep of random shapes through all three kernels against the float64 oracle.

Each case draws a batch of ragged sequences (empty ones included), a GQA ratio, a KV
dtype (bf16, fp16, e4m3fn or e5m2 with scales), causal or not, and a sliding window or
none. Slots are a random permutation of a shared pool, and the table rows are
permuted inside a larger ``req_to_token``. The same case runs through the split-KV
decode (the last token of each sequence), the split-KV verify (up to 16 rows per
sequence) and the MFMA extend (any number of rows). The sizes keep the oracle fast.
The head dim is 128 except in the ``headdim`` cases, which run 64 and 256, and the
``anydim`` cases, which run other multiples of 16 up to 512.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import attention as oracle
from tests.helpers import assert_attn_close, to_f64

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
KV = [torch.bfloat16, torch.float16, torch.float8_e4m3fn, torch.float8_e5m2]


def _ops():
    from sglang_restomod_amd.attention.mi355x import ops

    return ops


def _case(seed, max_q, dim=128, fp8=True):
    g = np.random.default_rng(seed)
    B = int(g.integers(1, 7))
    hkv = int(g.choice([1, 2, 4, 8]))
    G = int(g.choice([1, 2, 3, 5, 8]))
    kv = KV[int(g.integers(0, len(KV)))]
    if not fp8 and kv in KV[2:]:
        kv = KV[0] if kv == KV[2] else KV[1]
    q_dtype = torch.float16 if kv == torch.float16 else (torch.bfloat16 if kv == torch.bfloat16 else
                                                         (torch.float16 if g.random() < 0.3 else torch.bfloat16))
    prefix = [int(x) for x in g.integers(0, 700, B)]
    ext = [int(x) for x in g.integers(0, max_q + 1, B)]
    if sum(ext) == 0:
        ext[0] = 1
    causal = bool(g.random() < 0.8)
    window = int(g.choice([-1, -1, 0, 17, 100]))
    k_scale, v_scale = (float(g.uniform(0.5, 2)), float(g.uniform(0.5, 2))) if kv in KV[2:] else (1.0, 1.0)
    return B, hkv, G, kv, q_dtype, prefix, ext, causal, window, k_scale, v_scale


def _build(seed, max_q, dim=128, fp8=True):
    B, hkv, G, kv, q_dtype, prefix, ext, causal, window, ks, vs = _case(seed, max_q, dim, fp8)
    gen = torch.Generator().manual_seed(seed)
    seq = [p + e for p, e in zip(prefix, ext)]
    pool = sum(seq) + 64
    kf = torch.randn(pool, hkv, dim, generator=gen)
    vf = torch.randn(pool, hkv, dim, generator=gen)
    if kv in KV[2:]:
        k = (kf / ks).to(kv)
        v = (vf / vs).to(kv)
    else:
        k, v = kf.to(kv), vf.to(kv)
    T = sum(ext)
    q = torch.randn(T, hkv * G, dim, generator=gen).to(q_dtype)
    perm = torch.randperm(pool - 1, generator=gen) + 1
    rows = torch.randperm(B + 3, generator=gen)[:B]
    r2t = torch.zeros(B + 3, max(seq) + 5, dtype=torch.int32)
    off = 0
    for b, n in enumerate(seq):
        r2t[rows[b], :n] = perm[off:off + n].to(torch.int32)
        off += n
    qsl = [0] + list(np.cumsum(ext))
    case = dict(q=q, k=k, v=v, r2t=r2t, rows=rows, seq=seq, prefix=prefix, ext=ext, qsl=qsl, causal=causal,
                window=window, ks=ks, vs=vs, scale=dim ** -0.5)
    print(f"[case] seed={seed} D={dim} B={B} hkv={hkv} G={G} kv={kv} q={q_dtype} prefix={prefix} ext={ext} "
          f"causal={causal} window={window}", flush=True)
    return case


def _reference(c):
    kp = c["k"].float().numpy().astype(np.float64)
    vp = c["v"].float().numpy().astype(np.float64)
    slots = [c["r2t"][int(c["rows"][b]), :n].numpy().astype(np.int64) for b, n in enumerate(c["seq"])]
    return oracle.paged_attention(to_f64(c["q"]), kp, vp, slots, c["qsl"], c["prefix"], c["seq"],
                                  softmax_scale=c["scale"], k_scale=c["ks"], v_scale=c["vs"], causal=c["causal"],
                                  sliding_window=c["window"])


def _device(c):
    d = {n: c[n].to(DEV) for n in ("q", "k", "v", "r2t")}
    d["rows"] = c["rows"].to(torch.int64).to(DEV)
    d["seq"] = torch.tensor(c["seq"], dtype=torch.int32, device=DEV)
    d["qsl"] = torch.tensor(c["qsl"], dtype=torch.int32, device=DEV)
    d["pre"] = torch.tensor(c["prefix"], dtype=torch.int32, device=DEV)
    return d


def _run_extend(c):
    d = _device(c)
    out = _ops().paged_extend_forward(
        d["q"], d["k"], d["v"], d["r2t"], d["seq"], d["qsl"], d["pre"], softmax_scale=c["scale"],
        k_scale=c["ks"], v_scale=c["vs"], causal=c["causal"], sliding_window_size=c["window"], row_index=d["rows"])
    torch.cuda.synchronize()
    return out


def _run_verify(c):
    d = _device(c)
    out = _ops().paged_verify_forward(
        d["q"], d["k"], d["v"], d["r2t"], d["seq"], d["qsl"], d["pre"], max_q_per_seq=max(max(c["ext"]), 1),
        softmax_scale=c["scale"], k_scale=c["ks"], v_scale=c["vs"], causal=c["causal"],
        sliding_window_size=c["window"], row_index=d["rows"])
    torch.cuda.synchronize()
    return out


def _decode_case(seed, dim=128):
    c = _build(seed, max_q=1, dim=dim)
    # one query row per sequence, at its last position; empty sequences return zeros
    ctx = c["seq"]
    B, hq = len(ctx), c["q"].shape[1]
    gen = torch.Generator().manual_seed(seed)
    c["q"] = torch.randn(B, hq, dim, generator=gen).to(c["q"].dtype)
    c["qsl"] = list(range(B + 1))
    c["prefix"] = [max(n - 1, 0) for n in ctx]
    c["causal"] = True
    return c


def _run_decode(c):
    d = _device(c)
    out = _ops().grouped_decode_forward(
        d["q"], d["k"], d["v"], d["r2t"], d["seq"], softmax_scale=c["scale"], k_scale=c["ks"], v_scale=c["vs"],
        row_index=d["rows"], sliding_window_size=c["window"])
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("seed", range(12))
def test_sweep_extend(seed):
    c = _build(1000 + seed, max_q=200)
    assert_attn_close(_run_extend(c), _reference(c), what=f"extend seed {seed}")


@pytest.mark.parametrize("seed", range(12))
def test_sweep_verify(seed):
    c = _build(2000 + seed, max_q=16)
    assert_attn_close(_run_verify(c), _reference(c), what=f"verify seed {seed}")


@pytest.mark.parametrize("seed", range(12))
def test_sweep_decode(seed):
    c = _decode_case(3000 + seed)
    assert_attn_close(_run_decode(c), _reference(c), what=f"decode seed {seed}")


@pytest.mark.parametrize("dim", [64, 256])
@pytest.mark.parametrize("seed", range(6))
def test_sweep_headdim_extend(dim, seed):
    c = _build(4000 + seed, max_q=200, dim=dim)
    assert_attn_close(_run_extend(c), _reference(c), what=f"extend D={dim} seed {seed}")


@pytest.mark.parametrize("dim", [64, 256])
@pytest.mark.parametrize("seed", range(6))
def test_sweep_headdim_verify(dim, seed):
    c = _build(5000 + seed, max_q=16, dim=dim)
    assert_attn_close(_run_verify(c), _reference(c), what=f"verify D={dim} seed {seed}")


@pytest.mark.parametrize("dim", [64, 256])
@pytest.mark.parametrize("seed", range(6))
def test_sweep_headdim_decode(dim, seed):
    c = _decode_case(6000 + seed, dim=dim)
    assert_attn_close(_run_decode(c), _reference(c), what=f"decode D={dim} seed {seed}")


# Head dims outside 64/128/256: decode and verify run on the any-head-dim kernel (one wave
# per 16 rows, padded to the next of 64/128/256/512), extend up to 256 on the tiled extend
# kernel of the next of 64/128/256 and above on the any-head-dim kernel.
ANY_DIMS = [16, 48, 80, 96, 160, 192, 320, 448, 512]


@pytest.mark.parametrize("dim", ANY_DIMS)
@pytest.mark.parametrize("seed", range(2))
def test_sweep_anydim_extend(dim, seed):
    c = _build(7000 + 10 * ANY_DIMS.index(dim) + seed, max_q=200, dim=dim)
    assert_attn_close(_run_extend(c), _reference(c), what=f"extend D={dim} seed {seed}")


PADDED_DIMS = [d for d in range(16, 256, 16) if d not in (64, 128)]


@pytest.mark.parametrize("dim", PADDED_DIMS)
def test_sweep_every_padded_extend_dim(dim):
    """Every head dim that runs padded on a tiled extend kernel (16-48 on the 64 kernel,
    80-112 on 128, 144-240 on 256; 96 and 192 with their zero steps skipped). The seeded
    cases span all four KV dtypes, fp16 and bf16 queries, windows and non-causal rows."""
    seed = 9000 + dim
    c = _build(seed, max_q=120, dim=dim)
    assert_attn_close(_run_extend(c), _reference(c), what=f"extend D={dim}")


@pytest.mark.parametrize("dim", ANY_DIMS)
@pytest.mark.parametrize("seed", range(2))
def test_sweep_anydim_verify(dim, seed):
    c = _build(8000 + 10 * ANY_DIMS.index(dim) + seed, max_q=16, dim=dim)
    assert_attn_close(_run_verify(c), _reference(c), what=f"verify D={dim} seed {seed}")


@pytest.mark.parametrize("dim", ANY_DIMS)
@pytest.mark.parametrize("seed", range(2))
def test_sweep_anydim_decode(dim, seed):
    c = _decode_case(9000 + 10 * ANY_DIMS.index(dim) + seed, dim=dim)
    assert_attn_close(_run_decode(c), _reference(c), what=f"decode D={dim} seed {seed}")
