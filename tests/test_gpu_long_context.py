"""Long contexts and large batches through the tuned kernels against the float64 oracle.

The split-KV decode and verify cut every (sequence, kv head, row group) into 32-key tiles
(16 at D=256) and hand each wave of the persistent grid an equal range of the tile list,
so a sequence of 131,072 keys is shared by about a hundred waves and merged from as many
pieces; fp8 pools run the lazy rescale over the whole length. The extend kernel streams a
64k-key prefix through every row tile. A batch of 2,048 short sequences gives the decode
16,384 segments and the extend a work list of 2,048 row tiles; a batch of 128 with a
length bound of at most 512 keys runs the decode as one launch of the any-head-dim
kernel. Each case is seeded; slots are a random permutation of the pool and the request
rows are permuted inside a larger ``req_to_token``.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import attention as oracle
from tests.helpers import assert_attn_close, to_f64

pytestmark = pytest.mark.gpu

FP8 = (torch.float8_e4m3fn, torch.float8_e5m2)


def _ops():
    from sglang_restomod_amd.attention.mi355x import ops

    return ops


def _build(seed, prefix, ext, hkv, group, dim, kv, q_dtype):
    """Sequences of ``prefix[b] + ext[b]`` keys; ``ext[b]`` query rows each (the last ones)."""
    gen = torch.Generator().manual_seed(seed)
    B = len(prefix)
    seq = [p + e for p, e in zip(prefix, ext)]
    pool = sum(seq) + 8
    ks, vs = (1.25, 0.75) if kv in FP8 else (1.0, 1.0)
    kf = torch.randn(pool, hkv, dim, generator=gen)
    vf = torch.randn(pool, hkv, dim, generator=gen)
    k, v = ((kf / ks).to(kv), (vf / vs).to(kv)) if kv in FP8 else (kf.to(kv), vf.to(kv))
    T = sum(ext)
    q = torch.randn(T, hkv * group, dim, generator=gen).to(q_dtype)
    perm = torch.randperm(pool - 1, generator=gen) + 1
    rows = torch.randperm(B + 2, generator=gen)[:B]
    r2t = torch.zeros(B + 2, max(seq) + 5, dtype=torch.int32)
    off = 0
    for b, n in enumerate(seq):
        r2t[rows[b], :n] = perm[off:off + n].to(torch.int32)
        off += n
    shape = f"prefix={prefix} ext={ext}" if B <= 4 else f"batch={B} keys={sum(seq)} rows={T}"
    print(f"[case] long seed={seed} D={dim} {shape} hkv={hkv} G={group} kv={kv} q={q_dtype}", flush=True)
    return dict(q=q, k=k, v=v, r2t=r2t, rows=rows, seq=seq, prefix=prefix, ext=ext,
                qsl=[0] + list(np.cumsum(ext)), ks=ks, vs=vs, scale=dim ** -0.5)


def _reference(c, window=-1):
    slots = [c["r2t"][int(c["rows"][b]), :n].numpy().astype(np.int64) for b, n in enumerate(c["seq"])]
    kp = c["k"].float().numpy().astype(np.float64)
    vp = c["v"].float().numpy().astype(np.float64)
    return oracle.paged_attention(to_f64(c["q"]), kp, vp, slots, c["qsl"], c["prefix"], c["seq"],
                                  softmax_scale=c["scale"], k_scale=c["ks"], v_scale=c["vs"],
                                  sliding_window=window)


def _device(c, gpu):
    d = {n: c[n].to(gpu) for n in ("q", "k", "v", "r2t")}
    d["rows"] = c["rows"].to(torch.int64).to(gpu)
    d["seq"] = torch.tensor(c["seq"], dtype=torch.int32, device=gpu)
    d["qsl"] = torch.tensor(c["qsl"], dtype=torch.int32, device=gpu)
    d["pre"] = torch.tensor(c["prefix"], dtype=torch.int32, device=gpu)
    return d


def _decode(c, gpu, window=-1):
    d = _device(c, gpu)
    # no length hint: the persistent split-KV kernel, whatever the batch
    out = _ops().grouped_decode_forward(d["q"], d["k"], d["v"], d["r2t"], d["seq"], softmax_scale=c["scale"],
                                        k_scale=c["ks"], v_scale=c["vs"], row_index=d["rows"],
                                        sliding_window_size=window)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("window", [-1, 70_000])
def test_decode_131k_keys_bf16(gpu, window):
    c = _build(101, [131_071], [1], 8, 4, 128, torch.bfloat16, torch.bfloat16)
    assert_attn_close(_decode(c, gpu, window), _reference(c, window), what=f"decode 131k window {window}")


@pytest.mark.parametrize("kv", FP8)
def test_decode_131k_keys_fp8(gpu, kv):
    c = _build(102, [131_071, 65_536], [1, 1], 8, 4, 128, kv, torch.bfloat16)
    assert_attn_close(_decode(c, gpu), _reference(c), what=f"decode 131k {kv}")


def test_decode_65k_keys_head_dim_256(gpu):
    c = _build(103, [65_535, 9_000], [1, 1], 2, 6, 256, torch.bfloat16, torch.bfloat16)
    assert_attn_close(_decode(c, gpu), _reference(c), what="decode 65k D=256")


def test_verify_64k_prefix(gpu):
    c = _build(104, [65_536, 30_000], [4, 4], 8, 8, 128, torch.bfloat16, torch.bfloat16)
    d = _device(c, gpu)
    out = _ops().paged_verify_forward(d["q"], d["k"], d["v"], d["r2t"], d["seq"], d["qsl"], d["pre"],
                                      max_q_per_seq=4, softmax_scale=c["scale"], row_index=d["rows"])
    torch.cuda.synchronize()
    assert_attn_close(out, _reference(c), what="verify 64k prefix")


def test_extend_64k_prefix(gpu):
    c = _build(105, [65_536], [200], 8, 2, 128, torch.bfloat16, torch.bfloat16)
    d = _device(c, gpu)
    out = _ops().paged_extend_forward(d["q"], d["k"], d["v"], d["r2t"], d["seq"], d["qsl"], d["pre"],
                                      softmax_scale=c["scale"], row_index=d["rows"])
    torch.cuda.synchronize()
    assert_attn_close(out, _reference(c), what="extend 64k prefix")


def _ragged(seed, batch, lo, hi):
    g = np.random.default_rng(seed)
    return [int(x) for x in g.integers(lo, hi + 1, batch)]


@pytest.mark.parametrize("batch,hint", [(2048, False), (128, True)])
def test_decode_many_sequences(gpu, batch, hint):
    """2,048 sequences without a length hint: the persistent kernel over 16,384 segments.
    128 sequences with a hint of at most 512 keys: one launch of the any-head-dim kernel."""
    lens = _ragged(106, batch, 1, 100 if batch > 512 else 500)
    c = _build(106, [n - 1 for n in lens], [1] * len(lens), 8, 4, 128, torch.float16, torch.float16)
    d = _device(c, gpu)
    kw = {"max_seq_len_hint": max(lens)} if hint else {}
    out = _ops().grouped_decode_forward(d["q"], d["k"], d["v"], d["r2t"], d["seq"], softmax_scale=c["scale"],
                                        row_index=d["rows"], **kw)
    torch.cuda.synchronize()
    assert_attn_close(out, _reference(c), what=f"decode {batch} sequences hint={hint}")


def test_extend_2048_sequences(gpu):
    prefix = _ragged(107, 2048, 0, 100)
    ext = _ragged(108, 2048, 1, 40)
    c = _build(107, prefix, ext, 4, 4, 128, torch.bfloat16, torch.bfloat16)
    d = _device(c, gpu)
    out = _ops().paged_extend_forward(d["q"], d["k"], d["v"], d["r2t"], d["seq"], d["qsl"], d["pre"],
                                      softmax_scale=c["scale"], row_index=d["rows"])
    torch.cuda.synchronize()
    assert_attn_close(out, _reference(c), what="extend 2048 sequences")
