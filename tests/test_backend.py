"""The backend's engine-facing surface on the CPU: construction, mode routing,
per-forward metadata, graph-state buffers and the refusals. No kernel runs here:
a forward on CPU tensors must raise (there is no CPU path)."""

from __future__ import annotations

import pytest
import torch

from tests import fakes


def _backend(engine, **kw):
    from sglang_restomod_amd.attention.mi355x.backend import MI355XAttnBackend

    return MI355XAttnBackend(engine.runner, **kw)


def _engine(**kw):
    kw.setdefault("device", "cpu")
    return fakes.Engine(**kw)


def test_registry_factory_builds_the_backend():
    from sglang_restomod_amd.attention.mi355x import backend_registry
    from sglang_restomod_amd.attention.mi355x.backend import MI355XAttnBackend

    eng = _engine()
    be = backend_registry.build_backend(backend_registry.MI355X_ATTN, eng.runner)
    assert isinstance(be, MI355XAttnBackend)
    assert be.get_cuda_graph_seq_len_fill_value() == 1
    assert be.needs_cpu_seq_lens is False


@pytest.mark.parametrize("head_dim", [100, 528])
def test_unsupported_head_dim_is_refused_at_construction(head_dim):
    eng = _engine(head_dim=head_dim)
    with pytest.raises(NotImplementedError, match="head_dim"):
        _backend(eng)


@pytest.mark.parametrize("head_dim", [64, 128, 256, 16, 96, 192, 320, 512])
def test_supported_head_dims_construct(head_dim):
    be = _backend(_engine(head_dim=head_dim))
    assert be.head_dim == head_dim


def test_fp8_pool_at_head_dim_64_constructs():
    be = _backend(_engine(head_dim=64, kv_dtype=torch.float8_e4m3fn))
    assert be.head_dim == 64


def test_decode_metadata_uses_req_to_token_in_place():
    eng = _engine()
    eng.alloc(3, 17)
    eng.alloc(5, 40)
    be = _backend(eng)
    fb = eng.batch("DECODE", [5, 3], new_tokens=[1, 1])
    be.init_forward_metadata(fb)
    md = be.forward_metadata
    assert md.mode == "decode"
    assert md.table is eng.req_to_token  # no page table is built
    assert md.row_index.dtype == torch.int64 and md.row_index.tolist() == [5, 3]
    assert md.seq_lens.dtype == torch.int32 and md.seq_lens.tolist() == [41, 18]


def test_page_size_16_engine_places_positions_in_page_runs():
    """The fake engine at page size 16 (the reference's production page size): position p of
    a request lives at offset p % 16 of one page, pages are disjoint across requests, and
    the backend builds on it with the same token-level req_to_token metadata."""
    eng = _engine(page_size=16, pool_size=4096)
    eng.alloc(0, 40)
    eng.alloc(1, 5)
    eng.alloc(0, 9)   # continues request 0's third page, then opens a fourth
    eng.alloc(1, 30)
    seen = set()
    for row, n in ((0, 49), (1, 35)):
        slots = eng.req_to_token[row, :n].tolist()
        for p, s in enumerate(slots):
            assert s % 16 == p % 16 and s >= 16
            assert slots[p - p % 16] + p % 16 == s  # one page per 16 positions
        pages = {s // 16 for s in slots}
        assert len(pages) == -(-n // 16) and not (pages & seen)
        seen |= pages
    be = _backend(eng)
    assert be.page_size == 16
    fb = eng.batch("DECODE", [1, 0], new_tokens=[1, 1])
    be.init_forward_metadata(fb)
    md = be.forward_metadata
    assert md.table is eng.req_to_token and md.seq_lens.tolist() == [36, 50]
    assert eng.req_to_token[1, 35].item() % 16 == 35 % 16


def test_extend_metadata():
    eng = _engine()
    eng.alloc(0, 10)  # cached prefix of request 0
    be = _backend(eng)
    fb = eng.batch("EXTEND", [0, 1, 2], new_tokens=[5, 7, 1])
    be.init_forward_metadata(fb)
    md = be.forward_metadata
    assert md.mode == "extend"
    assert md.query_start_loc.tolist() == [0, 5, 12, 13]
    assert md.prefix_kv_lens.tolist() == [10, 0, 0]
    assert md.seq_lens.tolist() == [15, 7, 1]
    assert md.max_q_per_seq == 7
    assert md.query_start_loc.dtype == torch.int32


def test_extend_metadata_lifts_warmup_fill_value():
    """A warm-up batch with seq_lens = 1 still sees prefix + extend keys (reference :452-455)."""
    eng = _engine()
    be = _backend(eng)
    fb = eng.batch("EXTEND", [0, 1], new_tokens=[6, 3])
    fb.seq_lens = torch.ones(2, dtype=torch.int64)
    be.init_forward_metadata(fb)
    assert be.forward_metadata.seq_lens.tolist() == [6, 3]


def test_linear_verify_metadata():
    eng = _engine(spec="EAGLE", topk=1)
    eng.alloc(2, 30)
    eng.alloc(4, 9)
    be = _backend(eng)
    fb = eng.batch("TARGET_VERIFY", [2, 4], new_tokens=[4, 4], draft_token_num=4)
    be.init_forward_metadata(fb)
    md = be.forward_metadata
    assert md.mode == "verify"
    assert md.prefix_kv_lens.tolist() == [30, 9]
    assert md.seq_lens.tolist() == [34, 13]
    assert md.query_start_loc.tolist() == [0, 4, 8]
    assert md.max_q_per_seq == 4


def test_tree_verify_is_refused():
    eng = _engine(spec="EAGLE", topk=4)
    eng.alloc(0, 8)
    be = _backend(eng)
    fb = eng.batch("TARGET_VERIFY", [0], new_tokens=[4], draft_token_num=4)
    with pytest.raises(NotImplementedError, match="linear"):
        be.init_forward_metadata(fb)


def test_dflash_verify_is_linear_whatever_topk():
    eng = _engine(spec="DFLASH", topk=8)
    eng.alloc(0, 8)
    be = _backend(eng)
    be.init_forward_metadata(eng.batch("TARGET_VERIFY", [0], new_tokens=[4], draft_token_num=4))
    assert be.forward_metadata.mode == "verify"


@pytest.mark.parametrize("rows,mode", [(3, "verify"), (64, "verify"), (65, "extend")])
def test_draft_extend_routes_by_row_count(rows, mode):
    eng = _engine(spec="EAGLE", draft_worker=True)
    eng.alloc(0, 100)
    be = _backend(eng)
    be.init_forward_metadata(eng.batch("DRAFT_EXTEND_V2", [0], new_tokens=[rows]))
    assert be.forward_metadata.mode == mode


def test_draft_extend_routing_reads_no_device_value():
    """Without extend_seq_lens_cpu the route comes from the token and request counts, and
    the kernel's row-group hint from the token count; no device tensor is read."""
    eng = _engine(spec="EAGLE", draft_worker=True)
    eng.alloc(0, 50)
    eng.alloc(1, 60)
    be = _backend(eng)
    fb = eng.batch("DRAFT_EXTEND", [0, 1], new_tokens=[3, 2])
    del fb.extend_seq_lens_cpu

    class NoHostRead(torch.Tensor):
        def item(self):
            raise AssertionError("a device value was read on the host")

    fb.extend_seq_lens = fb.extend_seq_lens.as_subclass(NoHostRead)
    be.init_forward_metadata(fb)
    md = be.forward_metadata
    assert md.mode == "verify" and md.max_q_per_seq == 5  # 5 tokens in all: a bound of the longest chain
    assert md.query_start_loc.tolist() == [0, 3, 5]


@pytest.mark.parametrize("mode", ["DRAFT_EXTEND", "DRAFT_EXTEND_V2"])
def test_captured_draft_extend_uses_fixed_rows_per_request(mode):
    """A captured draft extend runs num_tokens / bs rows per request: request b's rows are
    the last n of its seq_lens[b] keys. Capture and replay fill the same device buffers;
    an uneven split is refused (it has no fixed layout)."""
    eng = _engine(spec="EAGLE", draft_worker=True)
    for r in range(3):
        eng.alloc(r, 40 + r)
    be = _backend(eng)
    be.init_cuda_graph_state(max_bs=4, max_num_tokens=16)
    fm = fakes.ForwardMode(mode)
    spec = type("S", (), {"draft_token_num": 4})()
    rpi, seq = torch.tensor([0, 1, 2]), torch.tensor([40, 41, 42])
    be.init_forward_metadata_capture_cuda_graph(3, 12, rpi, seq, None, fm, spec)
    md = be.forward_metadata
    assert md.mode == "verify" and md.max_q_per_seq == 4 and md.num_tokens == 12
    assert md.query_start_loc.tolist() == [0, 4, 8, 12]
    assert md.seq_lens.tolist() == [40, 41, 42] and md.prefix_kv_lens.tolist() == [36, 37, 38]
    ptrs = (md.seq_lens.data_ptr(), md.prefix_kv_lens.data_ptr(), md.query_start_loc.data_ptr())
    be.init_forward_metadata_replay_cuda_graph(3, torch.tensor([2, 0, 1]), torch.tensor([50, 44, 45]), 139,
                                               None, fm, spec, None)
    md = be.forward_metadata
    assert (md.seq_lens.data_ptr(), md.prefix_kv_lens.data_ptr(), md.query_start_loc.data_ptr()) == ptrs
    assert md.row_index.tolist() == [2, 0, 1] and md.num_tokens == 12
    assert md.seq_lens.tolist() == [50, 44, 45] and md.prefix_kv_lens.tolist() == [46, 40, 41]
    with pytest.raises(NotImplementedError, match="same number of rows"):
        be.init_forward_metadata_capture_cuda_graph(3, 10, rpi, seq, None, fm, spec)


def test_paged_forward_keeps_the_reference_signature():
    """Positional order and defaults of the reference's paged_forward
    (_paged_adapter.py:567-586); the extra keywords come after them."""
    import inspect

    from sglang_restomod_amd.attention.mi355x import ops

    params = list(inspect.signature(ops.paged_forward).parameters.values())
    ref = [("q", inspect.Parameter.empty), ("k_cache", inspect.Parameter.empty),
           ("v_cache", inspect.Parameter.empty), ("block_table", inspect.Parameter.empty),
           ("seq_lens", inspect.Parameter.empty), ("query_start_loc", inspect.Parameter.empty),
           ("prefix_kv_lens", inspect.Parameter.empty), ("out", None), ("block_size", 16),
           ("num_kv_heads", None), ("softmax_scale", None), ("causal", True), ("sliding_window_size", -1),
           ("linear_verify", False), ("k_scale", 1.0), ("v_scale", 1.0), ("max_seq_len_hint", None),
           ("logical_dense_kv", False)]
    assert [(p.name, p.default) for p in params[:len(ref)]] == ref


def test_graph_buffers_keep_their_addresses_across_replays():
    eng = _engine(spec="EAGLE")
    for r in range(4):
        eng.alloc(r, 10 + r)
    be = _backend(eng)
    be.init_cuda_graph_state(max_bs=8, max_num_tokens=32)
    mode = fakes.ForwardMode("DECODE")
    rpi = torch.tensor([3, 1, 0], dtype=torch.int64)
    be.init_forward_metadata_capture_cuda_graph(3, 3, rpi, torch.tensor([5, 6, 7]), None, mode, None)
    md0 = be.forward_metadata
    ptrs = (md0.seq_lens.data_ptr(), md0.row_index.data_ptr())
    be.init_forward_metadata_replay_cuda_graph(3, torch.tensor([2, 0, 1]), torch.tensor([9, 8, 7]), 24,
                                               None, mode, None, None)
    md1 = be.forward_metadata
    assert (md1.seq_lens.data_ptr(), md1.row_index.data_ptr()) == ptrs
    assert md1.seq_lens.tolist() == [9, 8, 7] and md1.row_index.tolist() == [2, 0, 1]
    # verify replay fills prefix, lengths and the start offsets in the same buffers
    vmode = fakes.ForwardMode("TARGET_VERIFY")
    spec = type("S", (), {"draft_token_num": 4})()
    be.init_forward_metadata_replay_cuda_graph(2, torch.tensor([1, 2]), torch.tensor([11, 12]), 23,
                                               None, vmode, spec, None)
    md2 = be.forward_metadata
    assert md2.mode == "verify" and md2.max_q_per_seq == 4
    assert md2.seq_lens.tolist() == [15, 16] and md2.prefix_kv_lens.tolist() == [11, 12]
    assert md2.query_start_loc.tolist() == [0, 4, 8]


def test_graph_batch_over_capacity_is_refused():
    eng = _engine()
    be = _backend(eng)
    be.init_cuda_graph_state(max_bs=2, max_num_tokens=2)
    with pytest.raises(ValueError, match="capacity"):
        be.init_forward_metadata_capture_cuda_graph(
            3, 3, torch.zeros(3, dtype=torch.int64), torch.ones(3), None, fakes.ForwardMode("DECODE"), None)


def test_swa_pool_rows_need_the_device():
    # the SWA table is translated by a HIP kernel; host tensors are refused, not served
    eng = _engine(swa=True)
    eng.alloc(1, 12)
    be = _backend(eng)
    with pytest.raises(ValueError, match="device tensors"):
        be.init_forward_metadata(eng.batch("DECODE", [1], new_tokens=[1]))


@pytest.mark.parametrize("attr,value,reason", [
    ("logit_cap", 30.0, "logit_cap"),
    ("is_cross_attention", True, "cross_attention"),
    ("xai_temperature_len", 8, "xai_temperature"),
])
def test_layers_the_kernels_cannot_serve_are_refused(attr, value, reason):
    eng = _engine()
    eng.alloc(0, 4)
    be = _backend(eng)
    fb = eng.batch("DECODE", [0], new_tokens=[1])
    be.init_forward_metadata(fb)
    layer = fakes.Layer(tp_q_head_num=8, tp_k_head_num=2)
    setattr(layer, attr, value)
    q = torch.zeros(1, 8 * 128, dtype=torch.bfloat16)
    with pytest.raises(NotImplementedError, match=reason):
        be.forward_decode(q, None, None, layer, fb, save_kv_cache=False)


def test_sinks_are_refused():
    eng = _engine()
    eng.alloc(0, 4)
    be = _backend(eng)
    fb = eng.batch("DECODE", [0], new_tokens=[1])
    be.init_forward_metadata(fb)
    layer = fakes.Layer(tp_q_head_num=8, tp_k_head_num=2)
    with pytest.raises(NotImplementedError, match="sinks"):
        be.forward_decode(torch.zeros(1, 1024, dtype=torch.bfloat16), None, None, layer, fb,
                          save_kv_cache=False, sinks=torch.zeros(8))


@pytest.mark.parametrize("native_write", ["1", "0"])
def test_forward_on_cpu_tensors_raises_instead_of_falling_back(native_write, monkeypatch):
    """The KV write and the attention both need device tensors: with the native write
    (the default) the write itself refuses; with the pool's own write the attention does."""
    monkeypatch.setenv("SGLANG_MI355X_NATIVE_KV_WRITE", native_write)
    eng = _engine()
    eng.alloc(0, 4)
    be = _backend(eng)
    assert be.native_kv_write == (native_write == "1")
    fb = eng.batch("DECODE", [0], new_tokens=[1])
    be.init_forward_metadata(fb)
    layer = fakes.Layer(tp_q_head_num=8, tp_k_head_num=2)
    q = torch.zeros(1, 8 * 128, dtype=torch.bfloat16)
    k = torch.zeros(1, 2, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="device tensors"):
        be.forward_decode(q, k, k.clone(), layer, fb)
    assert eng.pool.writes == (0 if native_write == "1" else 1)


def test_forward_without_metadata_raises():
    eng = _engine()
    be = _backend(eng)
    layer = fakes.Layer(tp_q_head_num=8, tp_k_head_num=2)
    fb = eng.batch("DECODE", [0], new_tokens=[1])
    with pytest.raises(RuntimeError, match="metadata"):
        be.forward_decode(torch.zeros(1, 1024), None, None, layer, fb, save_kv_cache=False)


def test_fake_pool_quantizes_like_the_token_pool():
    eng = _engine(kv_dtype=torch.float8_e4m3fn)
    layer = fakes.Layer(tp_q_head_num=8, tp_k_head_num=2, k_scale=torch.tensor(2.0), v_scale=torch.tensor(0.5))
    slots = eng.alloc(0, 3)
    k = torch.randn(3, 2, 128)
    eng.pool.set_kv_buffer(layer, slots, k, k, layer.k_scale, layer.v_scale)
    got = eng.pool.get_key_buffer(0)[slots].float()
    assert torch.equal(got, (k / 2.0).to(torch.float8_e4m3fn).float())
    assert eng.pool.k_buffer[0].dtype == torch.uint8
