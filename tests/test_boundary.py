"""Host-side boundary: plugin registry, attestation, backend registration, masks,
draft-decode planning. Mirrors the reference's CPU tests (tests/test_plugins.py,
test_attest.py, test_backend_registry.py, test_attention_v100.py:67-99,
test_native_draft_decode_plan.py) against this package."""

from __future__ import annotations

import json
import subprocess
import sys
import types

import pytest
import torch

from sglang_restomod_amd import attest, plugins
from sglang_restomod_amd.attention.mi355x import backend_registry, draft_decode_plan as plan
from sglang_restomod_amd.attention.mi355x.masks import resolve_layer_mask


# ---- plugins ----------------------------------------------------------------

def test_empty_selection():
    assert plugins.selection({}) == []
    assert plugins.selection({plugins.ENV_COMPONENTS: " , "}) == []


def test_parsing_and_dedup():
    env = {plugins.ENV_COMPONENTS: " attention_mi355x, attention_mi355x "}
    assert plugins.selection(env) == ["attention_mi355x"]


def test_unknown_component_lists_known_names():
    with pytest.raises(ValueError, match="unknown component.*known: attention_mi355x"):
        plugins.selection({plugins.ENV_COMPONENTS: "nope"})


def _fake_component(monkeypatch, name, module):
    monkeypatch.setitem(sys.modules, module.__name__, module)
    monkeypatch.setitem(plugins.COMPONENTS, name, plugins.Component(name, module.__name__, "test"))


def test_load_enabled_registers_once(monkeypatch):
    attest.reset()
    calls = []
    mod = types.ModuleType("ma_test_component")
    mod.register = lambda: calls.append(1)
    _fake_component(monkeypatch, "t1", mod)
    assert plugins.load_enabled({plugins.ENV_COMPONENTS: "t1"}) == ["t1"]
    assert calls == [1]
    assert attest.snapshot()["loaded"] == ["t1"]


def test_failures_are_recorded_and_the_rest_still_load(monkeypatch):
    attest.reset()
    no_reg = types.ModuleType("ma_no_register")
    bad = types.ModuleType("ma_bad_register")

    def boom():
        raise RuntimeError("kaput")

    bad.register = boom
    good = types.ModuleType("ma_good")
    good.register = lambda: None
    _fake_component(monkeypatch, "noreg", no_reg)
    _fake_component(monkeypatch, "bad", bad)
    _fake_component(monkeypatch, "good", good)
    monkeypatch.setitem(plugins.COMPONENTS, "missing",
                        plugins.Component("missing", "ma_module_that_does_not_exist", "x"))
    loaded = plugins.load_enabled({plugins.ENV_COMPONENTS: "noreg,bad,missing,good"})
    assert loaded == ["good"]
    snap = attest.snapshot()
    assert "has no register" in snap["components"]["noreg"]["detail"]
    assert snap["failed"] == ["bad"] and "kaput" in snap["components"]["bad"]["detail"]
    assert "import failed" in snap["components"]["missing"]["detail"]
    assert set(snap["inactive"]) == {"noreg", "missing"}
    attest.reset()


def test_plugin_import_is_light():
    code = ("import sys; import sglang_restomod_amd, sglang_restomod_amd.plugins; "
            "import sglang_restomod_amd.attention.mi355x.backend_registry; "
            "print('torch' in sys.modules)")
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, check=True,
                         cwd=__file__.rsplit("/tests/", 1)[0])
    assert out.stdout.strip() == "False"


# ---- attest -----------------------------------------------------------------

def test_attest_states_and_missing():
    attest.reset()
    attest.set_selected(["a", "b", "c"])
    attest.inactive("a", "no device")
    attest.record("a", True)  # keeps the inactive reason
    attest.record("b", False, "boom")
    snap = attest.snapshot()
    assert snap["components"]["a"]["detail"] == "registered, inactive: no device"
    assert snap["failed"] == ["b"] and snap["missing"] == ["c"]
    attest.reset()


def test_attest_write(tmp_path, monkeypatch):
    attest.reset()
    attest.set_selected(["x"])
    attest.record("x", True)
    target = tmp_path / "a.json"
    assert attest.write(str(target)) == str(target)
    assert json.loads(target.read_text())["loaded"] == ["x"]
    assert attest.write(str(tmp_path / "nodir" / "a.json")) is None  # swallowed
    monkeypatch.delenv(attest.ENV_ATTEST, raising=False)
    assert attest.write() is None
    attest.reset()


def test_attest_failure_after_inactive_and_list_order():
    attest.reset()
    attest.set_selected(["p", "q", "r"])
    attest.record("q", True)
    attest.inactive("p", "idle")
    attest.record("p", False, "broke later")
    attest.record("r", True, "fine")
    snap = attest.snapshot()
    assert snap["loaded"] == ["q", "r"] and snap["failed"] == ["p"] and snap["inactive"] == []
    assert snap["components"] == {"q": {"ok": True}, "p": {"ok": False, "detail": "broke later"},
                                  "r": {"ok": True, "detail": "fine"}}
    assert set(snap) == {"engine", "selected", "components", "loaded", "failed", "inactive", "missing"}
    attest.reset()


def test_attest_write_leaves_only_the_target(tmp_path):
    attest.reset()
    attest.set_selected(["x"])
    attest.inactive("x", object())
    target = tmp_path / "att.json"
    for _ in range(3):
        assert attest.write(str(target)) == str(target)
    assert [p.name for p in tmp_path.iterdir()] == ["att.json"]
    doc = json.loads(target.read_text())
    assert doc["inactive"] == ["x"] and doc["loaded"] == ["x"]
    assert doc["components"]["x"]["detail"].startswith("registered, inactive: ")
    attest.reset()


def test_register_entry_point_writes_attest(tmp_path, monkeypatch):
    import sglang_restomod_amd

    attest.reset()
    monkeypatch.setenv(attest.ENV_ATTEST, str(tmp_path / "att.json"))
    monkeypatch.setenv(plugins.ENV_COMPONENTS, "")
    sglang_restomod_amd.register()
    assert json.loads((tmp_path / "att.json").read_text())["selected"] == []
    attest.reset()


# ---- backend registration ---------------------------------------------------

def _fake_engine():
    registry, choices = {}, []

    def register(name):
        def deco(fn):
            registry[name] = fn
            return fn
        return deco

    return dict(registry=registry, register=register, choices=choices, extend_choices=choices.extend)


def test_install_registers_backend_and_choice():
    eng = _fake_engine()
    assert backend_registry.install(**eng, env={}) is True
    assert backend_registry.MI355X_ATTN in eng["registry"] and eng["choices"] == [backend_registry.MI355X_ATTN]


def test_install_is_idempotent():
    eng = _fake_engine()
    backend_registry.install(**eng, env={})
    assert backend_registry.install(**eng, env={}) is False
    assert eng["choices"].count(backend_registry.MI355X_ATTN) == 1


def test_v100_alias_is_opt_in():
    eng = _fake_engine()
    backend_registry.install(**eng, env={backend_registry.ENV_ALIAS: "1"})
    assert backend_registry.V100_ALIAS in eng["registry"]
    with pytest.raises(ValueError, match=backend_registry.ENV_ALIAS):
        backend_registry.backend_names({backend_registry.ENV_ALIAS: "maybe"})


def test_factory_does_not_import_the_backend_eagerly():
    code = ("import sys; from sglang_restomod_amd.attention.mi355x import backend_registry as r\n"
            "reg, ch = {}, []\n"
            "r.install(registry=reg, register=lambda n: (lambda f: reg.__setitem__(n, f)), choices=ch,"
            " extend_choices=ch.extend, env={})\n"
            "print('sglang_restomod_amd.attention.mi355x.backend' in sys.modules)")
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, check=True,
                         cwd=__file__.rsplit("/tests/", 1)[0])
    assert out.stdout.strip() == "False"


# ---- masks (reference tests/test_attention_v100.py:67-99) --------------------

def test_encoder_only_layer_keeps_its_window():
    assert resolve_layer_mask(default_causal=True, is_cross_attention=False, is_encoder_only=True,
                              sliding_window_size=2047) == (False, 2047)


def test_causal_layer_keeps_its_window():
    assert resolve_layer_mask(default_causal=True, is_cross_attention=False, is_encoder_only=False,
                              sliding_window_size=2047) == (True, 2047)


def test_layer_without_a_window_gets_minus_one():
    assert resolve_layer_mask(default_causal=True, is_cross_attention=False, is_encoder_only=True,
                              sliding_window_size=None) == (False, -1)


def test_cross_attention_is_not_causal():
    assert resolve_layer_mask(default_causal=True, is_cross_attention=True, is_encoder_only=False,
                              sliding_window_size=-5) == (False, -1)


# ---- draft decode planning (reference KATs) --------------------------------

def test_page_table_reads_the_page_start_of_each_row():
    row0 = [0, 1, 2, 3, 12, 13, 14, 15, 8]
    row1 = [20, 21, 22, 23, 4]
    kv_indices = torch.tensor(row0 + row1, dtype=torch.int64)
    kv_indptr = torch.tensor([0, 9, 14], dtype=torch.int32)
    table = torch.zeros((2, 3), dtype=torch.int32)
    seq = torch.zeros((2,), dtype=torch.int32)
    assert plan.page_table_from_indices(kv_indptr, kv_indices, table, seq, 4) == 2
    assert seq.tolist() == [9, 5] and table.tolist() == [[0, 3, 2], [5, 1, 0]]


def test_page_table_marks_unused_pages_zero():
    table = torch.full((2, 2), 7, dtype=torch.int32)
    seq = torch.zeros((2,), dtype=torch.int32)
    plan.page_table_from_indices(torch.tensor([0, 4, 4]), torch.arange(32), table, seq, 4)
    assert seq.tolist() == [4, 0] and table.tolist() == [[0, 0], [0, 0]]


def test_page_table_handles_an_empty_index_list():
    table = torch.full((1, 2), 5, dtype=torch.int32)
    seq = torch.ones((1,), dtype=torch.int32)
    assert plan.page_table_from_indices(torch.tensor([0, 1]), torch.empty(0, dtype=torch.int64), table, seq, 4) == 1
    assert seq.tolist() == [0] and table.tolist() == [[0, 0]]


def test_page_table_refuses_a_short_buffer():
    assert plan.page_table_from_indices(torch.tensor([0, 4, 8]), torch.arange(8),
                                        torch.zeros((1, 1), dtype=torch.int32), torch.zeros(1, dtype=torch.int32)) == 0


def test_page_table_matches_the_oracle_on_random_rows():
    from oracle import metadata as M

    g = torch.Generator().manual_seed(0)
    lens = [0, 1, 5, 17, 33]
    indptr = [0]
    for n in lens:
        indptr.append(indptr[-1] + n)
    idx = torch.randint(0, 1000, (indptr[-1],), generator=g)
    table = torch.full((6, 9), 3, dtype=torch.int32)
    seq = torch.zeros(6, dtype=torch.int32)
    rows = plan.page_table_from_indices(torch.tensor(indptr), idx, table, seq, 4)
    r2, t2, s2 = M.page_table_from_indices(indptr, idx.tolist(), 6, 9, 4)
    assert rows == r2 and table[:rows].tolist() == t2 and seq[:rows].tolist() == s2


class _Layer:
    def __init__(self, **kw):
        self.tp_q_head_num, self.tp_k_head_num = 40, 8
        self.qk_head_dim = self.v_head_dim = 128
        self.is_cross_attention = False
        self.sliding_window_size = None
        self.logit_cap = None
        self.xai_temperature_len = 0
        self.__dict__.update(kw)


def test_supported_layer_has_no_reason():
    assert plan.layer_shape_reason(_Layer()) is None
    assert plan.layer_shape_reason(_Layer(sliding_window_size=4096)) is None  # windows are served


@pytest.mark.parametrize("kw,reason", [
    ({"tp_k_head_num": 7}, "gqa_ratio"),
    ({"v_head_dim": 64}, "qk_dim"),
    ({"qk_head_dim": 250, "v_head_dim": 250}, "not_a_multiple"),
    ({"qk_head_dim": 528, "v_head_dim": 528}, "head_dim"),
    ({"is_cross_attention": True}, "cross_attention"),
    ({"logit_cap": 30.0}, "logit_cap"),
    ({"xai_temperature_len": 8}, "xai_temperature"),
])
def test_unsupported_layer_reports_the_reason(kw, reason):
    assert reason in plan.layer_shape_reason(_Layer(**kw))
