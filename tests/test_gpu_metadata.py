"""On-device metadata and the fp8 page gather on the GPU, bit-exact:

* ``translate_slots`` (the SWA table: req_to_token rows through the pool's
  full-to-SWA mapping, row by row up to each sequence's length) against numpy fancy
  indexing, with a row index, empty rows, rows longer than the width, slots outside
  the mapping, and positions past each length left untouched; also through the
  backend, eagerly and in a replayed HIP graph;
* ``gather_fp8_paged_kv`` against torch's own fp8 -> fp16 cast, which is the
  reference's lookup table (``_get_fp8_lut``, _paged_adapter.py:373-386): every one
  of the 256 codes of each format, bitwise for every non-NaN code and NaN for the NaN
  codes (the reference's own check, tests/test_e5m2_shift_lut.py:19-33: torch's cast
  canonicalises NaN payloads, the shift keeps them; for e5m2 the NaN outputs are also
  checked to be the shifted bytes), and the page placement of
  _kernels_fp8_bridge.py:55-70 (pages past a sequence's length untouched).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from tests import fakes

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
SENTINEL = -77


def _ops():
    from sglang_restomod_amd.attention.mi355x import ops

    return ops


def _translate_ref(table, seq, mapping, rows, width, out):
    out = out.copy()
    for b, r in enumerate(rows):
        n = min(int(seq[b]), width)
        slots = table[r, :n].astype(np.int64)
        ok = (slots >= 0) & (slots < len(mapping))
        out[b, :n] = np.where(ok, mapping[np.clip(slots, 0, len(mapping) - 1)], 0)
    return out


@pytest.mark.parametrize("with_rows", [True, False])
def test_translate_slots_matches_numpy(with_rows):
    g = torch.Generator().manual_seed(3)
    R, W, P = 9, 3000, 50_000
    table = torch.randint(0, P, (R, W), generator=g, dtype=torch.int32)
    table[2, 5] = P + 10        # outside the mapping -> 0
    table[4, 0] = -3            # negative -> 0
    mapping = torch.randint(0, 1 << 30, (P,), generator=g, dtype=torch.int64)
    rows = [4, 2, 7, 0, 8, 1] if with_rows else list(range(6))
    seq = [1, 2999, 0, 3000, 4100, 1030]   # an empty row, a row longer than the width
    width = W
    out0 = np.full((len(rows), width + 5), SENTINEL, dtype=np.int32)
    out = torch.from_numpy(out0).to(DEV)
    _ops().translate_slots(table.to(DEV), torch.tensor(seq, dtype=torch.int32, device=DEV), mapping.to(DEV),
                           row_index=torch.tensor(rows, device=DEV) if with_rows else None, out=out, width=width)
    torch.cuda.synchronize()
    want = _translate_ref(table.numpy(), seq, mapping.numpy(), rows, width, out0)
    np.testing.assert_array_equal(out.cpu().numpy(), want)


def test_translate_slots_through_the_backend_and_a_graph():
    from sglang_restomod_amd.attention.mi355x.backend import MI355XAttnBackend

    eng = fakes.Engine(DEV, hq=16, hkv=4, kv_dtype=torch.bfloat16, pool_size=4000, max_reqs=4,
                       context_len=1024, swa=True)
    for r, n in ((0, 300), (1, 17), (3, 900)):
        eng.alloc(r, n)
    be = MI355XAttnBackend(eng.runner)
    mapping = eng.pool.full_to_swa_index_mapping.cpu().numpy()

    def check(md, rows, lens):
        got = md.swa_table.cpu().numpy()
        r2t = eng.req_to_token.cpu().numpy()
        for b, (r, n) in enumerate(zip(rows, lens)):
            np.testing.assert_array_equal(got[b, :n], mapping[r2t[r, :n]])

    fb = eng.batch("DECODE", [3, 0, 1], new_tokens=[1, 1, 1])
    be.init_forward_metadata(fb)
    check(be.forward_metadata, [3, 0, 1], [901, 301, 18])
    be.init_cuda_graph_state(max_bs=3, max_num_tokens=3)
    rpi = torch.tensor([3, 0, 1], dtype=torch.int64, device=DEV)
    seq = torch.tensor([901, 301, 18], dtype=torch.int32, device=DEV)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        be.init_forward_metadata_capture_cuda_graph(3, 3, rpi, seq, None, fakes.ForwardMode("DECODE"), None)
    for it in range(3):
        for r in (3, 0, 1):
            eng.alloc(r, 5)
        seq.copy_(torch.tensor([eng.lens[3], eng.lens[0], eng.lens[1]], dtype=torch.int32))
        graph.replay()
        torch.cuda.synchronize()
        check(be.forward_metadata, [3, 0, 1], seq.tolist())


def _codes(fmt):
    return torch.arange(256, dtype=torch.uint8).view(fmt)


@pytest.mark.parametrize("fmt", [torch.float8_e4m3fn, torch.float8_e5m2])
def test_fp8_gather_decodes_every_code_like_the_cast(fmt):
    # one page of 16 tokens x 1 head x 16 dims holds all 256 codes
    k = _codes(fmt).view(1, 16, 1, 16)
    v = torch.arange(255, -1, -1, dtype=torch.int32).to(torch.uint8).view(fmt).view(1, 16, 1, 16)
    ko = torch.full((1, 16, 1, 16), -1.0, dtype=torch.float16, device=DEV)
    vo = torch.full_like(ko, -1.0)
    _ops().gather_fp8_paged_kv(k.to(DEV), v.to(DEV), torch.zeros(1, 1, dtype=torch.int32, device=DEV),
                               torch.tensor([16], dtype=torch.int32, device=DEV), ko, vo)
    torch.cuda.synchronize()
    for got, src in ((ko, k), (vo, v)):
        want = src.reshape(-1).to(torch.float16)           # the reference's lookup table
        g16, w16 = got.cpu().reshape(-1), want
        nan = torch.isnan(w16)
        assert torch.equal(torch.isnan(g16), nan)
        assert torch.equal(g16.view(torch.int16)[~nan], w16.view(torch.int16)[~nan])
        if fmt == torch.float8_e5m2:
            shifted = (src.reshape(-1).view(torch.uint8).to(torch.int32) << 8).to(torch.int16)
            assert torch.equal(g16.view(torch.int16), shifted)


def test_fp8_gather_places_logical_pages():
    g = torch.Generator().manual_seed(9)
    pages, ps, hkv, d = 40, 16, 8, 128
    fmt = torch.float8_e4m3fn
    k = torch.randint(0, 256, (pages, ps, hkv, d), generator=g, dtype=torch.uint8)
    k[k == 0x7F] = 0
    k[k == 0xFF] = 0
    v = torch.randint(0, 256, (pages, ps, hkv, d), generator=g, dtype=torch.uint8)
    v[(v & 0x7F) == 0x7F] = 1
    B, max_blocks = 3, 5
    table = torch.tensor([[7, 3, 39, 0, 11], [20, 21, 22, 23, 24], [5, 6, 0, 0, 0]], dtype=torch.int32)
    seq = [33, 80, 0]                       # 3 pages, 5 pages, none
    ko = torch.full((B * max_blocks, ps, hkv, d), 7.0, dtype=torch.float16, device=DEV)
    vo = torch.full_like(ko, 7.0)
    _ops().gather_fp8_paged_kv(k.view(fmt).to(DEV), v.view(fmt).to(DEV), table.to(DEV),
                               torch.tensor(seq, dtype=torch.int32, device=DEV), ko, vo)
    torch.cuda.synchronize()
    kf, vf = k.view(fmt).to(torch.float16), v.view(fmt).to(torch.float16)
    want_k = torch.full_like(ko.cpu(), 7.0)
    want_v = torch.full_like(vo.cpu(), 7.0)
    for b in range(B):
        for p in range((seq[b] + ps - 1) // ps):
            want_k[b * max_blocks + p] = kf[table[b, p]]
            want_v[b * max_blocks + p] = vf[table[b, p]]
    assert torch.equal(ko.cpu().view(torch.int16), want_k.view(torch.int16))
    assert torch.equal(vo.cpu().view(torch.int16), want_v.view(torch.int16))


def test_fp8_gather_rejects_a_16_bit_cache():
    x = torch.zeros(1, 16, 1, 16, dtype=torch.float16, device=DEV)
    with pytest.raises(ValueError, match="E4M3 or E5M2"):
        _ops().gather_fp8_paged_kv(x, x, torch.zeros(1, 1, dtype=torch.int32, device=DEV),
                                   torch.ones(1, dtype=torch.int32, device=DEV), x, x)
