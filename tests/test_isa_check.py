"""The build's static checks of generated assembly fire on planted listings (CPU only)."""

from __future__ import annotations

from sglang_restomod_amd import isa_check

KERNEL = """_ZN2ma15splitkv_partialEv:
{body}
.Lfunc_end0:
"""


def _write(tmp_path, body):
    p = tmp_path / "k.s"
    p.write_text(KERNEL.format(body=body))
    return str(p)


def test_register_read_before_its_wait_is_a_hazard(tmp_path):
    body = "\tglobal_load_dwordx4 a[0:3], v[2:3], off\n\tv_mov_b32 v9, a1\n\ts_waitcnt vmcnt(0)\n"
    assert isa_check.check_file(_write(tmp_path, body)) > 0


def test_register_read_after_its_wait_is_clean(tmp_path):
    body = "\tglobal_load_dwordx4 a[0:3], v[2:3], off\n\ts_waitcnt vmcnt(0)\n\tv_mov_b32 v9, a1\n"
    assert isa_check.check_file(_write(tmp_path, body)) == 0


def test_in_order_counting_keeps_later_loads_in_flight(tmp_path):
    body = ("\tglobal_load_dwordx4 a[0:3], v[2:3], off\n\tglobal_load_dwordx4 a[4:7], v[2:3], off\n"
            "\ts_waitcnt vmcnt(1)\n\tv_mov_b32 v9, a1\n\tv_mov_b32 v10, a5\n\ts_waitcnt vmcnt(0)\n")
    # only the read of a5 is a hazard
    assert isa_check.check_file(_write(tmp_path, body)) == 1


def test_load_pending_across_a_loop_back_edge_is_a_hazard(tmp_path):
    # the next iteration reads a1 before waiting for the previous iteration's load
    body = (".LBB0_1:\n\tv_mov_b32 v9, a1\n\tglobal_load_dwordx4 a[0:3], v[2:3], off\n"
            "\ts_cbranch_scc1 .LBB0_1\n\ts_waitcnt vmcnt(0)\n\ts_endpgm\n")
    assert isa_check.check_file(_write(tmp_path, body)) == 1


def test_a_later_load_into_the_same_register_is_in_order(tmp_path):
    body = ("\tglobal_load_dwordx4 v[2:5], v[8:9], off\n\tscratch_load_dword v5, off, off offset:4\n"
            "\ts_waitcnt vmcnt(0)\n\tv_mov_b32 v9, v5\n")
    assert isa_check.check_file(_write(tmp_path, body)) == 0


def test_a_load_whose_address_is_in_flight_is_a_hazard(tmp_path):
    body = ("\tglobal_load_dwordx2 v[2:3], v[8:9], off\n\tglobal_load_dword v5, v[2:3], off\n"
            "\ts_waitcnt vmcnt(0)\n")
    assert isa_check.check_file(_write(tmp_path, body)) == 1


def test_wait_at_the_loop_top_retires_the_load(tmp_path):
    body = (".LBB0_1:\n\ts_waitcnt vmcnt(0)\n\tv_mov_b32 v9, a1\n\tglobal_load_dwordx4 a[0:3], v[2:3], off\n"
            "\ts_cbranch_scc1 .LBB0_1\n\ts_waitcnt vmcnt(0)\n\ts_endpgm\n")
    assert isa_check.check_file(_write(tmp_path, body)) == 0


def test_out_of_line_block_is_checked_in_execution_order(tmp_path):
    # .LBB0_2 is laid out after the load but runs before it: no hazard
    body = ("\ts_cbranch_scc1 .LBB0_2\n.LBB0_1:\n\tglobal_load_dword v7, v[2:3], off\n"
            "\ts_waitcnt vmcnt(0)\n\tv_mov_b32 v9, v7\n\ts_endpgm\n"
            ".LBB0_2:\n\tv_mov_b32 v7, 1.0\n\ts_branch .LBB0_1\n")
    assert isa_check.check_file(_write(tmp_path, body)) == 0


def test_scalar_cache_writes_are_found(tmp_path):
    body = "\ts_store_dword s0, s[2:3], 0x0\n\ts_dcache_wb\n\tglobal_store_dword v0, v1, s[0:1]\n"
    found = isa_check.scalar_cache_writes(_write(tmp_path, body))
    assert len(found) == 2 and all(f.startswith("s_") for f in found)


def test_built_library_sources_are_clean():
    import glob
    import os

    build = os.path.join(os.path.dirname(isa_check.__file__), "csrc", "_build")
    listings = glob.glob(os.path.join(build, "*.s"))
    for path in listings:
        assert isa_check.scalar_cache_writes(path) == [], path
