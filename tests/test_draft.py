"""Draft-worker plumbing on the CPU: the factory patch, the launch gate, the multi-step
container over a stand-in for the engine's container, and a step's metadata."""

from __future__ import annotations

from types import SimpleNamespace

import pytest
import torch

from sglang_restomod_amd.attention.mi355x import draft_backend, draft_decode, draft_decode_plan
from tests import fakes


class Factory:
    """Stand-in for the engine's DraftBackendFactory."""

    def __init__(self, name, steps=3, topk=1):
        self.draft_attn_backend = name
        self.speculative_num_steps = steps
        self.topk = topk
        self.draft_model_runner = "runner"
        self.calls = []

    def create_draft_extend_backend(self):
        self.calls.append(("extend", self.draft_attn_backend))
        return "engine-extend"

    def create_decode_backend(self):
        self.calls.append(("decode", self.draft_attn_backend))
        return "engine-decode"


def _patched(native="native"):
    cls = type("F", (Factory,), {})
    built = []
    wrapped = SimpleNamespace()
    changed = draft_backend.install_on(
        cls, build=lambda r: built.append(r) or "backend", wrap=lambda r, b: wrapped,
        build_native=lambda r, topk, steps, stamp: native)
    return cls, built, wrapped, changed


def test_other_names_keep_the_engine_backends():
    cls, built, _, _ = _patched()
    f = cls("triton")
    assert f.create_draft_extend_backend() == "engine-extend"
    assert f.create_decode_backend() == "engine-decode"
    assert built == []


def test_draft_extend_gets_the_backend_wrapped_and_stamped():
    cls, built, wrapped, changed = _patched()
    assert changed
    f = cls("mi355x_attn")
    assert f.create_draft_extend_backend() is wrapped
    assert built == ["runner"]
    assert wrapped.prefill_attention_backend_str == "mi355x_attn"


def test_draft_decode_gets_the_native_container():
    cls, _, _, _ = _patched(native="native-container")
    assert cls("mi355x_attn", steps=3).create_decode_backend() == "native-container"


def test_unsupported_draft_decode_falls_back_and_restores_the_name():
    cls, _, _, _ = _patched(native=None)
    f = cls("mi355x_attn", steps=3)
    assert f.create_decode_backend() == "engine-decode"
    assert f.calls[-1] == ("decode", "triton")
    assert f.draft_attn_backend == "mi355x_attn"


def test_single_step_draft_uses_the_engine_decode():
    cls, _, _, _ = _patched()
    f = cls("mi355x_attn", steps=1)
    assert f.create_decode_backend() == "engine-decode"


def test_patching_twice_changes_nothing():
    cls, _, _, _ = _patched()
    assert draft_backend.install_on(cls, build=None, wrap=None) is False


def _runner(**over):
    eng = fakes.Engine("cpu")
    r = eng.runner
    r.model_config.dtype = torch.bfloat16
    for k, v in over.items():
        setattr(r, k, v)
    return r


LAYERS = [fakes.Layer(8, 2)]


@pytest.mark.parametrize("over,env,window,layers,reason", [
    ({}, {"SGLANG_MI355X_DRAFT_DECODE_NATIVE": "0"}, (0, 0), LAYERS, "disabled_by_env"),
    ({"page_size": 16}, {}, (0, 0), LAYERS, "page_size"),
    ({"kv_cache_dtype": torch.float32}, {}, (0, 0), LAYERS, "kv_dtype"),
    ({}, {}, (128, 0), LAYERS, "draft_window"),
    ({"sliding_window_size": 512}, {}, (0, 0), LAYERS, "draft_sliding_window"),
    ({"kv_index_translator": SimpleNamespace(is_translating=True)}, {}, (0, 0), LAYERS, "kv_index_translation"),
    ({}, {}, (0, 0), [], "no_attention_layers"),
    ({}, {}, (0, 0), [fakes.Layer(8, 2, head_dim=96)], "head_dim"),
])
def test_unsupported_reasons(over, env, window, layers, reason):
    got = draft_decode.unsupported_reason(_runner(**over), 1, env=env, draft_window=window, layers=layers)
    assert got is not None and reason in got


def test_supported_launch_has_no_reason():
    assert draft_decode.unsupported_reason(_runner(), 1, env={}, layers=LAYERS) is None


def test_swa_pool_is_refused():
    eng = fakes.Engine("cpu", swa=True)
    eng.runner.model_config.dtype = torch.bfloat16
    assert draft_decode.unsupported_reason(eng.runner, 1, env={}, layers=LAYERS) == "swa_kv_pool"


class EngineContainer:
    """Stand-in for the engine's TritonMultiStepDraftBackend."""

    def __init__(self, model_runner, topk, speculative_num_steps):
        self.max_context_len = 2048
        self.speculative_num_steps = speculative_num_steps
        self.topk = topk
        self.templates = []

    def common_template(self, forward_batch, kv_indices_buffer, call_fn):
        self.templates.append(forward_batch)
        for step in range(self.speculative_num_steps - 1):
            call_fn(step, forward_batch)

    def init_forward_metadata_out_graph(self, forward_batch, in_capture=False):
        return "captured"


def test_container_has_split_kv_children_and_replays_through_the_template():
    runner = _runner()
    runner.model = SimpleNamespace(modules=lambda: list(LAYERS))
    cont = draft_decode.build_native(runner, 1, 4, "mi355x_attn", base_cls=EngineContainer)
    assert len(cont.attn_backends) == 3
    assert all(isinstance(c, draft_decode.MI355XDraftDecodeBackend) for c in cont.attn_backends)
    assert cont.decode_attention_backend_str == "mi355x_attn"
    indptr = torch.tensor([0, 3, 5], dtype=torch.int32)
    indices = torch.tensor([7, 8, 9, 1, 2], dtype=torch.int32)
    fb = SimpleNamespace(spec_info=SimpleNamespace(kv_indptr=indptr, kv_indices=indices))
    assert cont.init_forward_metadata_out_graph(fb, in_capture=True) == "captured"
    cont.init_forward_metadata_out_graph(fb, in_capture=False)
    assert cont.templates == [fb]
    assert all(c._rows_used == 2 for c in cont.attn_backends)


def test_step_metadata_reads_the_flat_list_in_place():
    runner = _runner()
    step = draft_decode.MI355XDraftDecodeBackend(runner, 2, 2048, 1, 3)
    indptr = torch.tensor([0, 4, 4, 7], dtype=torch.int32)
    indices = torch.tensor([5, 6, 7, 8, 10, 11, 12], dtype=torch.int32)
    assert step.refresh(indptr, indices) == 3
    assert step._row_index.tolist() == [0, 4, 4] and step._row_index.dtype == torch.int64
    assert step._seq_lens.tolist() == [4, 0, 3] and step._seq_lens.dtype == torch.int32
    # position p of row r is table[row_index[r] * 1 + p]
    assert step._table.stride() == (1, 1) and step._table.data_ptr() == indices.data_ptr()
    assert [int(step._table[int(step._row_index[2]) + p, 0]) for p in range(3)] == [10, 11, 12]


def test_step_metadata_in_graph_buffers_keeps_addresses():
    runner = _runner()
    step = draft_decode.MI355XDraftDecodeBackend(runner, 1, 2048, 1, 3)
    step.init_cuda_graph_state(max_bs=4, max_num_tokens=4)
    step.refresh(torch.tensor([0, 2, 5], dtype=torch.int32), torch.arange(5, dtype=torch.int32))
    p = (step._row_index.data_ptr(), step._seq_lens.data_ptr())
    step.refresh(torch.tensor([0, 1, 2], dtype=torch.int32), torch.arange(2, dtype=torch.int32))
    assert (step._row_index.data_ptr(), step._seq_lens.data_ptr()) == p
    assert step._seq_lens.tolist() == [1, 1]
    with pytest.raises(ValueError, match="capacity"):
        step.refresh(torch.arange(7, dtype=torch.int32), torch.arange(6, dtype=torch.int32))


def test_step_sizes_its_workspace_for_the_model_head_dim():
    """The split-KV workspace grows with the head dim, so a step takes the model's
    (and the largest supported one when the runner gives no model config)."""
    runner = _runner()
    runner.model_config.head_dim = 256
    assert draft_decode.MI355XDraftDecodeBackend(runner, 1, 2048, 1, 3).head_dim == 256
    bare = SimpleNamespace(**{k: v for k, v in vars(_runner()).items() if k != "model_config"})
    step = draft_decode.MI355XDraftDecodeBackend(bare, 1, 2048, 1, 3)
    assert step.head_dim == max(draft_decode_plan.SUPPORTED_HEAD_DIMS)


def test_step_refuses_mismatched_rows():
    step = draft_decode.MI355XDraftDecodeBackend(_runner(), 1, 2048, 1, 3)
    step.refresh(torch.tensor([0, 2], dtype=torch.int32), torch.arange(2, dtype=torch.int32))
    with pytest.raises(RuntimeError, match="rows"):
        step.forward_decode(torch.zeros(3, 8 * 128), None, None, fakes.Layer(8, 2), None, save_kv_cache=False)
