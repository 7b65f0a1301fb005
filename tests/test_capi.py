"""The C-ABI library: builds, loads, exports every symbol include/*.h declares, and
rejects bad arguments before launching anything (no GPU needed for these)."""

from __future__ import annotations

import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    names = []
    inc = os.path.join(ROOT, "include")
    for f in sorted(os.listdir(inc)):
        if f.endswith(".h"):
            text = open(os.path.join(inc, f)).read()
            text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
            names += re.findall(r"\b(ma_[a-z0-9_]+)\s*\(", text)
    return sorted(set(names))


@pytest.fixture(scope="module")
def lib():
    from sglang_restomod_amd.attention.mi355x import _lib

    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail(f"{_lib.LIB_PATH} is not built (run __graft_entry__.build())")
    return _lib.load()


def test_every_declared_symbol_is_exported(lib):
    names = _declared()
    assert "ma_grouped_decode" in names and "ma_last_error" in names
    for name in names:
        assert hasattr(lib, name), f"{name} declared in include/ but not exported"


def test_python_signatures_cover_the_header():
    from sglang_restomod_amd.attention.mi355x import _lib

    assert set(_declared()) == set(_lib.SIGNATURES)


def test_abi_version(lib):
    hdr = open(os.path.join(ROOT, "include", "mi355x_attn.h")).read()
    want = int(re.search(r"#define MA_ABI_VERSION (\d+)", hdr).group(1))
    assert lib.ma_abi_version() == want


def _decode_args(**over):
    args = dict(q=1 << 20, qs0=1024, qs1=128, qdt=1, k=1 << 21, v=1 << 22, rs=1024, hs=128, kvdt=1,
                table=1 << 23, tstride=64, rowidx=None, ps=1, seq=1 << 24, batch=2, hq=8, hkv=8, dim=128,
                nwg=4, sm=0.1, ks=1.0, vs=1.0, win=-1, msl=0, ws=None, wsb=0,
                out=1 << 25, odt=1, os0=1024, os1=128, stream=None)
    args.update(over)
    return list(args.values())


@pytest.mark.parametrize("over,msg", [
    ({"dim": 100}, "head_dim"),
    ({"dim": 528}, "head_dim"),
    ({"qdt": 2}, "q dtype"),
    ({"kvdt": 0}, "16-bit KV dtype must equal"),
    ({"hq": 12, "hkv": 8}, "head counts"),
    ({"ps": 3}, "power of two"),
    ({"sm": 0.0}, "scale"),
    ({"q": (1 << 20) + 2}, "aligned"),
    ({"ws": None, "wsb": 0}, "workspace"),
    ({"ws": 1 << 26, "wsb": 1024}, "workspace too small"),
    ({"nwg": 0}, "num_workgroups"),
    ({"odt": 2}, "out dtype"),
    ({"odt": 4, "os1": 130}, "aligned"),
    ({"msl": -1}, "max_seq_len"),
    ({"rs": 1 << 31}, "exceeds 4 GiB"),  # bf16 rows of 4 GiB: the kernels' 32-bit row stride
])
def test_bad_arguments_are_rejected_before_launch(lib, over, msg):
    status = lib.ma_grouped_decode(*_decode_args(**over))
    assert status != 0
    assert msg in lib.ma_last_error().decode()


def test_empty_batch_is_a_no_op(lib):
    assert lib.ma_grouped_decode(*_decode_args(batch=0)) == 0


def test_workspace_size_formula(lib):
    assert lib.ma_splitkv_workspace_bytes(0, 128) == 0
    # the other head dims hold only the key pieces of a split decode: two per compute unit,
    # 16 rows each, at the kernel's padded width (O) plus one LSE per row
    for d, dp in ((16, 64), (96, 128), (192, 256), (320, 512), (512, 512)):
        n = lib.ma_splitkv_workspace_bytes(256, d)
        assert n == 512 * 16 * dp * 4 + 512 * 16 * 4, d
    n = lib.ma_splitkv_workspace_bytes(256, 128)
    # two partial pieces of up to 32 rows per wave, 4 waves per workgroup
    assert n >= 256 * 4 * 2 * 32 * 129 * 4 and n % 256 == 0
    # which also hold the pieces of a small decode routed to the any-head-dim kernel
    assert n >= 512 * 16 * 128 * 4 + 512 * 16 * 4


def _kvw_args(**over):
    args = dict(k=1 << 20, v=1 << 21, sst=1024, ssh=128, sdt=1, loc=1 << 22, T=4, hkv=8, dim=128,
                kc=1 << 23, vc=1 << 24, crs=1024, chs=128, cdt=2, slots=100, ks=1.0, vs=1.0, apply=1,
                stream=None)
    args.update(over)
    return list(args.values())


@pytest.mark.parametrize("over,msg", [
    ({"sdt": 2}, "source dtype"),
    ({"cdt": 7}, "cache dtype"),
    ({"dim": 100}, "multiple of 8"),
    ({"dim": 4096}, "multiple of 8"),
    ({"ks": 0.0}, "positive"),
    ({"k": (1 << 20) + 4}, "aligned"),
    ({"sst": 1001}, "source strides"),
    ({"hkv": 0}, "bad sizes"),
])
def test_kv_write_rejects_bad_arguments(lib, over, msg):
    assert lib.ma_set_kv_buffer(*_kvw_args(**over)) != 0
    assert msg in lib.ma_last_error().decode()


def test_kv_write_of_nothing_is_a_no_op(lib):
    assert lib.ma_set_kv_buffer(*_kvw_args(T=0)) == 0


def _extend_args(**over):
    args = dict(q=1 << 20, qs0=1024, qs1=128, qdt=1, T=64, k=1 << 21, v=1 << 22, rs=1024, hs=128, kvdt=1,
                table=1 << 23, tstride=64, rowidx=None, ps=1, seq=1 << 24, qsl=1 << 25, pre=None,
                batch=2, hq=16, hkv=2, dim=128, causal=1, win=-1, sm=0.1, ks=1.0, vs=1.0,
                ws=1 << 26, wsb=1 << 12, out=1 << 27, odt=1, os0=1024, os1=128, stream=None)
    args.update(over)
    return list(args.values())


@pytest.mark.parametrize("over,msg", [
    ({"dim": 100}, "head_dim"),
    ({"dim": 528}, "head_dim"),
    ({"qdt": 3}, "q dtype"),
    ({"kvdt": 0}, "16-bit KV dtype must equal"),
    ({"hq": 12, "hkv": 8}, "head counts"),
    ({"ps": 6}, "power of two"),
    ({"sm": -1.0}, "scale"),
    ({"T": -1}, "num_tokens"),
    ({"batch": 16385}, "exceeds"),
    ({"out": (1 << 27) + 8}, "aligned"),
    ({"ws": None}, "workspace too small"),
    ({"wsb": 8}, "workspace too small"),
    ({"ws": (1 << 26) + 64}, "256-byte aligned"),
    ({"odt": 0}, "out dtype"),
    ({"odt": 4, "os0": 1026}, "aligned"),
])
def test_extend_rejects_bad_arguments(lib, over, msg):
    assert lib.ma_paged_extend(*_extend_args(**over)) != 0
    assert msg in lib.ma_last_error().decode()


def test_extend_of_nothing_is_a_no_op(lib):
    assert lib.ma_paged_extend(*_extend_args(T=0)) == 0
    assert lib.ma_paged_extend(*_extend_args(batch=0)) == 0


def test_extend_workspace_covers_every_row_tile(lib):
    # sized for the smallest row tile (128 rows, head dim 256), which covers every head dim:
    # sum over sequences of ceil(E_b * G / 128) <= ceil(T * G / 128) + B
    assert lib.ma_extend_workspace_bytes(1000, 40, 8, 3) == ((40 + 3) * 8 + 255) // 256 * 256
    assert lib.ma_extend_workspace_bytes(100000, 64, 8, 300) == ((6250 + 300) * 8 + 255) // 256 * 256
    assert lib.ma_extend_workspace_bytes(10, 12, 8, 1) == 0


@pytest.mark.parametrize("over,msg", [
    ({"batch": -1}, ">= 0"),
    ({"batch": 70000}, "65535"),
    ({"ostride": 10, "width": 20}, "out_stride"),
    ({"mapping": None}, "null pointer"),
])
def test_translate_slots_rejects_bad_arguments(lib, over, msg):
    args = dict(table=1 << 20, tstride=64, rowidx=None, seq=1 << 21, batch=2, mapping=1 << 22, mlen=100,
                out=1 << 23, ostride=64, width=64, stream=None)
    args.update(over)
    assert lib.ma_translate_slots(*args.values()) != 0
    assert msg in lib.ma_last_error().decode()


def test_translate_slots_of_nothing_is_a_no_op(lib):
    assert lib.ma_translate_slots(None, 0, None, None, 0, None, 0, None, 0, 8, None) == 0


def _g8_args(**over):
    args = dict(k=1 << 20, v=1 << 21, sp=16 * 8 * 128, st=8 * 128, sh=128, dt=2, pages=10, table=1 << 22,
                tstride=4, seq=1 << 23, batch=2, maxb=4, ps=16, hkv=8, dim=128, ko=1 << 24, vo=1 << 25,
                stream=None)
    args.update(over)
    return list(args.values())


@pytest.mark.parametrize("over,msg", [
    ({"dt": 1}, "e4m3 or e5m2"),
    ({"dim": 72}, "multiple of 16"),
    ({"ps": 0}, "bad sizes"),
    ({"ko": (1 << 24) + 8}, "aligned"),
    ({"st": 1000}, "aligned"),
    ({"tstride": 3}, "stride"),
])
def test_fp8_gather_rejects_bad_arguments(lib, over, msg):
    assert lib.ma_gather_fp8_paged_kv(*_g8_args(**over)) != 0
    assert msg in lib.ma_last_error().decode()


def test_loader_constants_match_the_header():
    import pathlib

    from sglang_restomod_amd.attention.mi355x import _lib as L

    hdr = (pathlib.Path(__file__).resolve().parents[1] / "include" / "mi355x_attn.h").read_text()
    for name in ("MA_OK", "MA_EINVAL", "MA_ELAUNCH", "MA_EUNSUPPORTED", "MA_NOALLOC_MAX_WORKGROUPS"):
        want = int(re.search(rf"#define {name} \(?(-?\d+)\)?", hdr).group(1))
        assert getattr(L, name) == want, name


def test_small_decode_rule_matches_the_library():
    """ops.decode_kernel mirrors the library's routing constant and rule."""
    from sglang_restomod_amd.attention.mi355x import ops

    src = open(os.path.join(ROOT, "sglang_restomod_amd", "csrc", "splitkv.hip")).read()
    assert int(re.search(r"#define MA_SMALL_DECODE_TILES (\d+)", src).group(1)) == ops.SMALL_DECODE_TILES
    assert ops.decode_kernel(1, 32, 8, 128, 512) == "any_kernel"          # 8 x 16 tiles
    assert ops.decode_kernel(1, 32, 8, 128, None) == "splitkv_partial"    # no bound: persistent
    assert ops.decode_kernel(64, 64, 8, 128, 8192) == "splitkv_partial"
    assert ops.decode_kernel(64, 16, 4, 512, 8192) == "any_kernel"        # not a tuned head dim
    assert ops.decode_kernel(8, 64, 8, 128, 8192) == "any_kernel"         # 8 x 8 x 256 = 16384 tiles
    assert ops.decode_kernel(8, 64, 8, 128, 8193) == "splitkv_partial"
