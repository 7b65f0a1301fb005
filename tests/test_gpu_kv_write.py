"""ma_set_kv_buffer against the KV-write oracle, bit-exact over every 16-bit input."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import kv_write as KW

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
TORCH = {"bf16": torch.bfloat16, "fp16": torch.float16, KW.E4M3: torch.float8_e4m3fn, KW.E5M2: torch.float8_e5m2}
ALL16 = np.arange(65536, dtype=np.uint32).astype(np.uint16)


def _ops():
    from sglang_restomod_amd.attention.mi355x import ops

    return ops


def _src(bits, dt, heads=1, dim=128):
    t = torch.from_numpy(bits.astype(np.int16).copy()).view(TORCH[dt])
    return t.view(-1, heads, dim).to(DEV)


def _nan_code(codes, dst):
    return ((codes & 0x7F) == 0x7F) if dst == KW.E4M3 else ((codes & 0x7F) > 0x7C)


def _cache(slots, heads, dim, dt):
    if dt in (KW.E4M3, KW.E5M2):
        return torch.zeros(slots, heads, dim, dtype=torch.uint8, device=DEV).view(TORCH[dt])
    return torch.zeros(slots, heads, dim, dtype=TORCH[dt], device=DEV)


def _bits(cache, dt):
    if dt in (KW.E4M3, KW.E5M2):
        return cache.view(torch.uint8).cpu().numpy()
    return cache.view(torch.int16).cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("src", ["bf16", "fp16"])
@pytest.mark.parametrize("dst", [KW.E4M3, KW.E5M2])
@pytest.mark.parametrize("scale", [None, 1.0, 0.37, 2.5])
def test_every_16bit_input_is_quantized_like_the_oracle(src, dst, scale):
    gen = torch.Generator().manual_seed(5)
    k = _src(ALL16, src)                      # 512 rows of 128
    v = _src(ALL16[::-1].copy(), src)
    T = k.shape[0]
    loc = torch.randperm(600, generator=gen)[:T].to(DEV)
    kc, vc = _cache(600, 1, 128, dst), _cache(600, 1, 128, dst)
    _ops().set_kv_buffer(kc, vc, loc, k, v, scale, None if scale is None else 1.5 * scale)
    torch.cuda.synchronize()
    loc_np = loc.cpu().numpy()
    for cache, bits, sc in ((kc, ALL16, scale), (vc, ALL16[::-1].copy(), None if scale is None else 1.5 * scale)):
        got = _bits(cache, dst)[loc_np].reshape(-1)
        want = KW.quantize(bits, src, dst, sc)
        nan_in = np.isnan(KW.source_values(bits, src))
        bad = np.nonzero((got != want) & ~nan_in)[0]
        assert bad.size == 0, [(hex(int(bits[i])), hex(int(got[i])), hex(int(want[i]))) for i in bad[:8]]
        assert _nan_code(got[nan_in], dst).all()
        untouched = np.setdiff1d(np.arange(600), loc_np)
        assert (_bits(cache, dst)[untouched] == 0).all()


@pytest.mark.parametrize("src", ["bf16", "fp16"])
def test_same_dtype_is_an_exact_copy(src):
    k = _src(ALL16, src)
    loc = torch.arange(k.shape[0], device=DEV).flip(0)
    kc, vc = _cache(k.shape[0], 1, 128, src), _cache(k.shape[0], 1, 128, src)
    _ops().set_kv_buffer(kc, vc, loc, k, k, 0.5, 0.5)  # scales are ignored for a same-dtype pool
    torch.cuda.synchronize()
    got = _bits(kc, src)[loc.cpu().numpy()].reshape(-1)
    assert (got == ALL16).all()


def test_bf16_into_fp16_pool_with_scale():
    k = _src(ALL16, "bf16")
    loc = torch.arange(k.shape[0], device=DEV)
    kc, vc = _cache(k.shape[0], 1, 128, "fp16"), _cache(k.shape[0], 1, 128, "fp16")
    _ops().set_kv_buffer(kc, vc, loc, k, k, 0.75, 0.75)
    torch.cuda.synchronize()
    got = _bits(kc, "fp16").reshape(-1)
    want = KW.quantize(ALL16, "bf16", "fp16", 0.75)
    ok = (got == want) | (np.isnan(KW.source_values(ALL16, "bf16")))
    assert ok.all()


def test_strided_rows_heads_and_out_of_pool_slots():
    gen = torch.Generator().manual_seed(9)
    T, H, D = 37, 8, 128
    qkv = torch.randn(T, (16 + 2 * H) * D, generator=gen).to(torch.bfloat16).to(DEV)
    k = qkv[:, 16 * D:(16 + H) * D].view(T, H, D)          # strided views of a fused projection
    v = qkv[:, (16 + H) * D:].view(T, H, D)
    loc = torch.randperm(100, generator=gen)[:T].to(DEV)
    loc[3] = 100      # past the pool: skipped
    loc[5] = -1       # negative: skipped
    kc, vc = _cache(100, H, D, KW.E4M3), _cache(100, H, D, KW.E4M3)
    _ops().set_kv_buffer(kc, vc, loc, k, v, 0.8, 1.2)
    torch.cuda.synchronize()
    loc_np = loc.cpu().numpy()
    kb = k.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
    vb = v.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
    for t in range(T):
        if not 0 <= loc_np[t] < 100:
            continue
        assert (_bits(kc, KW.E4M3)[loc_np[t]] == KW.quantize(kb[t], "bf16", KW.E4M3, 0.8)).all()
        assert (_bits(vc, KW.E4M3)[loc_np[t]] == KW.quantize(vb[t], "bf16", KW.E4M3, 1.2)).all()
    written = set(int(x) for x in loc_np if 0 <= x < 100)
    others = [s for s in range(100) if s not in written]
    assert (_bits(kc, KW.E4M3)[others] == 0).all()


@pytest.mark.parametrize("dim", [24, 96, 200, 520])
@pytest.mark.parametrize("dst", [KW.E4M3, "bf16"])
def test_head_dims_that_are_not_powers_of_two(dim, dst):
    """Rows of any multiple of 8 (the any-head-dim layers' pools): bit-exact over the 16-bit
    inputs that fill whole rows, untouched slots stay zero."""
    gen = torch.Generator().manual_seed(dim)
    heads = 2
    n = ALL16.size // (heads * dim)
    bits = ALL16[:n * heads * dim]
    k = _src(bits, "bf16", heads=heads, dim=dim)
    v = _src(bits[::-1].copy(), "bf16", heads=heads, dim=dim)
    loc = torch.randperm(n + 50, generator=gen)[:n].to(DEV)
    kc, vc = _cache(n + 50, heads, dim, dst), _cache(n + 50, heads, dim, dst)
    _ops().set_kv_buffer(kc, vc, loc, k, v, 0.37, 2.5)
    torch.cuda.synchronize()
    loc_np = loc.cpu().numpy()
    for cache, b, sc in ((kc, bits, 0.37), (vc, bits[::-1].copy(), 2.5)):
        got = _bits(cache, dst)[loc_np].reshape(-1)
        want = KW.quantize(b, "bf16", dst, sc if dst != "bf16" else None)
        nan_in = np.isnan(KW.source_values(b, "bf16"))
        bad = np.nonzero((got != want) & ~nan_in)[0]
        assert bad.size == 0, (dim, dst, bad[:8])
        untouched = np.setdiff1d(np.arange(n + 50), loc_np)
        assert (_bits(cache, dst)[untouched] == 0).all()
