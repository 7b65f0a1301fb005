"""Draft-worker plumbing on the CPU: the factory routing, the support gate, the multi-step
container's per-round rows (top-k 1 over req_to_token in place, graph buffers), and a
pass's flat-list rows."""

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


def _rerouted(container="container"):
    cls = type("F", (Factory,), {})
    built, made = [], []
    wrapped = SimpleNamespace()

    def build_container(runner, topk, steps, name):
        made.append((runner, topk, steps, name))
        if isinstance(container, Exception):
            raise container
        return container

    changed = draft_backend.install_on(cls, build=lambda r: built.append(r) or "backend", wrap=lambda r, b: wrapped,
                                       build_container=build_container)
    return cls, built, wrapped, made, changed


def test_other_names_keep_the_engine_backends():
    cls, built, _, made, _ = _rerouted()
    f = cls("triton")
    assert f.create_draft_extend_backend() == "engine-extend"
    assert f.create_decode_backend() == "engine-decode"
    assert built == [] and made == []


def test_draft_extend_gets_the_backend_wrapped_and_stamped():
    cls, built, wrapped, _, changed = _rerouted()
    assert changed
    f = cls("mi355x_attn")
    assert f.create_draft_extend_backend() is wrapped
    assert built == ["runner"]
    assert wrapped.prefill_attention_backend_str == "mi355x_attn"
    assert wrapped.decode_attention_backend_str == "mi355x_attn"


def test_draft_decode_gets_the_split_kv_container():
    cls, _, _, made, _ = _rerouted(container="native-container")
    assert cls("mi355x_attn", steps=3, topk=2).create_decode_backend() == "native-container"
    assert made == [("runner", 2, 3, "mi355x_attn")]


def test_unservable_draft_decode_raises_instead_of_rerouting():
    cls, _, _, _, _ = _rerouted(container=NotImplementedError("no"))
    f = cls("mi355x_attn", steps=3)
    with pytest.raises(NotImplementedError):
        f.create_decode_backend()
    assert f.calls == []  # nothing was handed to the engine's own backends
    assert f.draft_attn_backend == "mi355x_attn"


def test_single_step_draft_uses_the_engine_method():
    cls, _, _, made, _ = _rerouted()
    f = cls("mi355x_attn", steps=1)
    assert f.create_decode_backend() == "engine-decode"
    assert made == []


def test_rerouting_twice_changes_nothing_and_uninstall_restores():
    cls, _, _, _, _ = _rerouted()
    assert draft_backend.install_on(cls, build=None, wrap=None) is False
    assert draft_backend.uninstall(cls) is True
    assert cls("mi355x_attn").create_decode_backend() == "engine-decode"
    assert draft_backend.uninstall(cls) is False


def test_no_triton_anywhere_in_the_package():
    import pathlib

    pkg = pathlib.Path(draft_backend.__file__).resolve().parents[2]
    hits = [str(p) for p in pkg.rglob("*") if p.suffix in (".py", ".hip", ".h") and "triton" in p.read_text().lower()]
    assert hits == []


def _runner(**over):
    eng = fakes.Engine("cpu")
    r = eng.runner
    r.model_config.dtype = torch.bfloat16
    for k, v in over.items():
        setattr(r, k, v)
    return r


LAYERS = [fakes.Layer(8, 2)]


@pytest.mark.parametrize("over,topk,window,layers,gap", [
    ({"page_size": 16}, 2, (0, 0), LAYERS, "page size 16"),
    ({"kv_cache_dtype": torch.float32}, 1, (0, 0), LAYERS, "KV cache dtype"),
    ({}, 1, (128, 0), LAYERS, "draft-decode window"),
    ({}, 1, (0, 4), LAYERS, "sink=4"),
    ({"kv_index_translator": SimpleNamespace(is_translating=True)}, 1, (0, 0), LAYERS, "KV index translation"),
    ({}, 1, (0, 0), [fakes.Layer(8, 2, head_dim=100)], "dim(100)_not_a_multiple_of_16"),
    ({}, 1, (0, 0), [fakes.Layer(8, 2, head_dim=528)], "head_dim(528)"),
    ({}, 1, (0, 0), [fakes.Layer(8, 3)], "gqa_ratio"),
])
def test_support_gaps(over, topk, window, layers, gap):
    gaps = draft_decode.support_gaps(_runner(**over), topk, window, layers)
    assert any(gap in g for g in gaps), gaps
    with pytest.raises(NotImplementedError, match="cannot serve this draft worker"):
        draft_decode.MI355XMultiStepDraftBackend(_runner(**over), topk, 3, draft_window=window, layers=layers)


@pytest.mark.parametrize("over,topk", [({}, 1), ({"page_size": 16}, 1), ({}, 4), ({"sliding_window_size": 512}, 1)])
def test_servable_draft_workers(over, topk):
    assert draft_decode.support_gaps(_runner(**over), topk, (0, 0), LAYERS) == []


def test_swa_pool_is_served():
    eng = fakes.Engine("cpu", swa=True)
    eng.runner.model_config.dtype = torch.bfloat16
    assert draft_decode.support_gaps(eng.runner, 1, (0, 0), LAYERS) == []


def _container(steps=4, topk=1, **eng_kw):
    eng = fakes.Engine("cpu", **eng_kw)
    eng.runner.model_config.dtype = torch.bfloat16
    return eng, draft_decode.MI355XMultiStepDraftBackend(eng.runner, topk, steps, layers=LAYERS)


def test_container_children_and_stamps():
    _, cont = _container(steps=4)
    assert len(cont.attn_backends) == 3 and cont.passes == 3
    assert [c.step for c in cont.attn_backends] == [0, 1, 2]
    assert all(c.decode_attention_backend_str == "mi355x_attn" for c in (cont, *cont.attn_backends))


def test_top1_round_reads_req_to_token_in_place():
    """With one branch the draft tokens follow the prefix in req_to_token, so every pass
    reads the request's own row: pass i sees seq_len + i + 1 keys."""
    eng, cont = _container(steps=4, topk=1)
    fb = SimpleNamespace(req_pool_indices=torch.tensor([3, 1]), seq_lens=torch.tensor([10, 25]), batch_size=2,
                         seq_lens_cpu=torch.tensor([10, 25]))
    cont.init_forward_metadata(fb)
    rows = cont.current
    assert rows.table is eng.req_to_token
    assert rows.row_index.tolist() == [3, 1]
    assert rows.lens.tolist() == [[11, 26], [12, 27], [13, 28]]
    assert rows.swa_table is None
    assert all(c.rows() is rows for c in cont.attn_backends)


def test_graph_round_keeps_buffer_addresses():
    _, cont = _container(steps=3, topk=1)
    cont.init_cuda_graph_state(max_bs=4, max_num_tokens=4)
    fb = SimpleNamespace(req_pool_indices=torch.tensor([0, 2, 1]), seq_lens=torch.tensor([5, 6, 7]), batch_size=3)
    cont.init_forward_metadata_capture_cuda_graph(fb)
    ptrs = (cont.current.row_index.data_ptr(), cont.current.lens.data_ptr())
    fb2 = SimpleNamespace(req_pool_indices=torch.tensor([1, 0, 2]), seq_lens=torch.tensor([9, 3, 4]), batch_size=3)
    cont.init_forward_metadata_replay_cuda_graph(fb2, 3)
    assert (cont.current.row_index.data_ptr(), cont.current.lens.data_ptr()) == ptrs
    assert cont.current.row_index.tolist() == [1, 0, 2]
    assert cont.current.lens.tolist() == [[10, 4, 5], [11, 5, 6]]
    with pytest.raises(ValueError, match="capacity"):
        cont.plan(torch.arange(5), torch.ones(5, dtype=torch.int32), graph=True)


def test_flat_list_rows_are_read_in_place():
    indptr = torch.tensor([0, 4, 4, 7], dtype=torch.int32)
    indices = torch.tensor([5, 6, 7, 8, 10, 11, 12], dtype=torch.int32)
    rows = draft_decode.DraftRows.from_flat_lists(indptr, indices)
    assert rows.rows == 3
    assert rows.row_index.tolist() == [0, 4, 4] and rows.row_index.dtype == torch.int64
    assert rows.lens.tolist() == [[4, 0, 3]] and rows.lens.dtype == torch.int32
    # position p of row r is table[row_index[r] * 1 + p]
    assert rows.table.stride() == (1, 1) and rows.table.data_ptr() == indices.data_ptr()
    assert [int(rows.table[int(rows.row_index[2]) + p, 0]) for p in range(3)] == [10, 11, 12]


def test_flat_list_rows_over_an_swa_pool_translate_for_window_layers():
    """A pass fed by a flat list over an SWA pool: sliding-window layers read the list
    translated into SWA slots (same row starts), full-attention layers the list itself."""
    eng, cont = _container(steps=3, swa=True)
    mapping = eng.pool.full_to_swa_index_mapping
    indptr = torch.tensor([0, 3, 5], dtype=torch.int32)
    indices = torch.tensor([7, 2, 9, 4, 11], dtype=torch.int32)
    child = cont.attn_backends[1]
    assert child.use_flat_lists(indptr, indices) == 2
    rows = child.rows()
    assert rows.swa_table is not None and rows.swa_row_index.tolist() == [0, 3]
    full_t, full_r = child.table_for(rows, -1)
    assert full_t.data_ptr() == indices.data_ptr() and full_r.tolist() == [0, 3]
    swa_t, swa_r = child.table_for(rows, 64)
    assert swa_r.tolist() == [0, 3]
    got = [int(swa_t[int(swa_r[r]) + p, 0]) for r, n in ((0, 3), (1, 2)) for p in range(n)]
    assert got == mapping[indices.long()].tolist()
    # a full-attention pool keeps one table for every layer
    _, plain = _container(steps=3)
    plain.attn_backends[0].use_flat_lists(indptr, indices)
    r2 = plain.attn_backends[0].rows()
    assert r2.swa_table is None and plain.attn_backends[0].table_for(r2, 64)[0].data_ptr() == indices.data_ptr()


def test_eager_rounds_reuse_one_table_buffer():
    """Top-k > 1 eager rounds write their rows into one container buffer, sized by the
    longest row when the host has the lengths, and reused by later rounds."""
    eng, cont = _container(steps=3, topk=2, context_len=2048)
    seen = []
    for lens in ([10, 25], [12, 27], [5, 6]):
        fb = SimpleNamespace(req_pool_indices=torch.tensor([3, 1]), seq_lens=torch.tensor(lens), batch_size=2,
                             seq_lens_cpu=torch.tensor(lens))
        try:
            cont.init_forward_metadata(fb)
        except ValueError:  # the table kernel needs device tensors; the buffer is chosen first
            pass
        buf = cont._eager["table"]
        seen.append(buf.data_ptr())
        assert buf.shape[0] == 4 and buf.shape[1] <= max(max(x) for x in ([10, 25], [12, 27])) + 3
    assert len(set(seen[1:])) == 1


def test_pass_refuses_mismatched_rows():
    _, cont = _container(steps=3)
    cont.attn_backends[0].use_flat_lists(torch.tensor([0, 2], dtype=torch.int32), torch.arange(2, dtype=torch.int32))
    with pytest.raises(RuntimeError, match="rows"):
        cont.attn_backends[0].forward_decode(torch.zeros(3, 8 * 128), None, None, fakes.Layer(8, 2), None,
                                             save_kv_cache=False)


def test_container_sizes_its_workspace_for_the_model_head_dim():
    eng = fakes.Engine("cpu", head_dim=256)
    eng.runner.model_config.dtype = torch.bfloat16
    cont = draft_decode.MI355XMultiStepDraftBackend(eng.runner, 1, 3, layers=[fakes.Layer(8, 2, head_dim=256)])
    assert cont.head_dim == 256
    bare = SimpleNamespace(**{k: v for k, v in vars(_runner()).items() if k != "model_config"})
    # without a model head dim: the one with the largest split-KV workspace
    assert draft_decode.MI355XMultiStepDraftBackend(bare, 1, 3, layers=LAYERS).head_dim == 256
