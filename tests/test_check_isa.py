"""The build-time check of asynchronous LDS reads (flashprefillv2-mlx_amd/check_isa.py).

Synthetic gfx950 assembly: each case plants one of the mistakes the checker
exists to catch (a register of an in-flight read touched before its wait on
some path through the branches, loops included, or a read in flight at the
end) next to the accepted forms.
"""

from __future__ import annotations

import sys
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parents[1] / "flashprefillv2-mlx_amd"))

import check_isa  # noqa: E402


def _fn(body: str) -> str:
    return "k_sparse_attn_kernel_case:\n" + body + "\ts_endpgm\n.Lfunc_end0:\n"


def test_register_parsing():
    assert check_isa._regs("v[80:83], v84 offset:0") == {("v", r) for r in (80, 81, 82, 83, 84)}
    assert check_isa._regs("a[0:1], v7") == {("a", 0), ("a", 1), ("v", 7)}
    assert check_isa._regs("s[4:5], vcc") == set()


def test_use_after_wait_is_accepted():
    text = _fn("\tds_read_b128 v[80:83], v84 offset:0\n\ts_waitcnt lgkmcnt(0)\n"
               "\tv_mov_b32_e32 v1, v81\n")
    assert check_isa.check_text(text) == []


def test_use_before_wait_is_rejected():
    text = _fn("\tds_read_b128 v[80:83], v84 offset:0\n\tv_mov_b32_e32 v1, v81\n"
               "\ts_waitcnt lgkmcnt(0)\n")
    errors = check_isa.check_text(text)
    assert len(errors) == 1 and "v_mov_b32_e32 v1, v81" in errors[0]


def test_spill_of_in_flight_register_is_rejected():
    text = _fn("\tds_read_b64_tr_b16 v[10:11], v2 offset:64\n"
               "\tscratch_store_dword off, v11, off offset:8\n\ts_waitcnt lgkmcnt(0)\n")
    assert len(check_isa.check_text(text)) == 1


def test_counted_waits_retire_in_order():
    ok = _fn("\tds_read_b128 v[80:83], v84\n\tds_read_b128 v[90:93], v84 offset:32\n"
             "\ts_waitcnt lgkmcnt(1)\n\tv_mov_b32_e32 v1, v81\n\ts_waitcnt lgkmcnt(0)\n"
             "\tv_mov_b32_e32 v1, v91\n")
    bad = _fn("\tds_read_b128 v[80:83], v84\n\tds_read_b128 v[90:93], v84 offset:32\n"
              "\ts_waitcnt lgkmcnt(1)\n\tv_mov_b32_e32 v1, v91\n\ts_waitcnt lgkmcnt(0)\n")
    assert check_isa.check_text(ok) == []
    assert len(check_isa.check_text(bad)) == 1


def test_scalar_load_outstanding_leaves_the_youngest_reads():
    # lgkmcnt(1) with a scalar load in flight may retire the scalar load
    # instead of the LDS read ...
    text = _fn("\ts_load_dword s4, s[0:1], 0x0\n\tds_read_b128 v[80:83], v84\n"
               "\ts_waitcnt lgkmcnt(1)\n\tv_mov_b32_e32 v1, v81\n\ts_waitcnt lgkmcnt(0)\n")
    assert len(check_isa.check_text(text)) == 1
    # ... but at most one operation of any kind is then outstanding, so
    # every LDS read but the youngest has completed
    ok = _fn("\ts_load_dword s4, s[0:1], 0x0\n\tds_read_b128 v[80:83], v84\n"
             "\tds_read_b128 v[90:93], v84 offset:32\n\ts_waitcnt lgkmcnt(1)\n"
             "\tv_mov_b32_e32 v1, v81\n\ts_waitcnt lgkmcnt(0)\n")
    assert check_isa.check_text(ok) == []


def test_read_in_flight_around_a_loop_is_followed():
    # the back-edge carries the read into the next iteration, whose read of
    # the same registers lands while it is still in flight
    bad = _fn(".LBB0_1:\n\tds_read_b128 v[80:83], v84\n\ts_cbranch_scc1 .LBB0_1\n"
              "\ts_waitcnt lgkmcnt(0)\n")
    assert any("ds_read_b128 v[80:83]" in e for e in check_isa.check_text(bad))
    # waited for at the top of the next iteration: accepted
    ok = _fn(".LBB0_1:\n\ts_waitcnt lgkmcnt(0)\n\tv_mov_b32_e32 v1, v81\n"
             "\tds_read_b128 v[80:83], v84\n\ts_cbranch_scc1 .LBB0_1\n\ts_waitcnt lgkmcnt(0)\n")
    assert check_isa.check_text(ok) == []


def test_each_path_to_a_use_must_wait():
    # the taken branch skips the wait that the fall-through has
    bad = _fn("\tds_read_b128 v[80:83], v84\n\ts_cbranch_scc1 .LBB0_2\n\ts_waitcnt lgkmcnt(0)\n"
              ".LBB0_2:\n\tv_mov_b32_e32 v1, v81\n")
    assert any("v_mov_b32_e32 v1, v81" in e for e in check_isa.check_text(bad))
    ok = _fn("\tds_read_b128 v[80:83], v84\n\ts_cbranch_scc1 .LBB0_2\n\ts_waitcnt lgkmcnt(0)\n"
             "\ts_branch .LBB0_3\n.LBB0_2:\n\ts_waitcnt lgkmcnt(0)\n.LBB0_3:\n"
             "\tv_mov_b32_e32 v1, v81\n")
    assert check_isa.check_text(ok) == []


def test_backward_jump_within_one_pass_is_followed():
    # a block laid out above its predecessor: the jump back carries the read
    # in flight, and the target waits for it
    ok = _fn("\tds_read_b128 v[80:83], v84\n\ts_cbranch_scc1 .LBB0_2\n.LBB0_1:\n"
             "\ts_waitcnt lgkmcnt(0)\n\tv_mov_b32_e32 v1, v81\n\ts_branch .LBB0_3\n"
             ".LBB0_2:\n\ts_branch .LBB0_1\n.LBB0_3:\n")
    assert check_isa.check_text(ok) == []
    bad = _fn("\tds_read_b128 v[80:83], v84\n\ts_cbranch_scc1 .LBB0_2\n\ts_waitcnt lgkmcnt(0)\n"
              ".LBB0_1:\n\tv_mov_b32_e32 v1, v81\n\ts_branch .LBB0_3\n"
              ".LBB0_2:\n\ts_branch .LBB0_1\n.LBB0_3:\n")
    assert any("v_mov_b32_e32 v1, v81" in e for e in check_isa.check_text(bad))


def test_read_in_flight_at_end_is_rejected():
    text = _fn("\tds_read_b128 v[80:83], v84\n")
    assert any("s_endpgm" in e for e in check_isa.check_text(text))


def test_other_functions_are_ignored():
    text = ("other_kernel:\n\tds_read_b128 v[80:83], v84\n\tv_mov_b32_e32 v1, v81\n"
            "\ts_endpgm\n.Lfunc_end0:\n")
    assert check_isa.check_text(text) == []


def test_lds_write_may_stay_in_flight_across_back_edge():
    # a write has no destination registers: only reads must be waited for;
    # the write still counts in the in-order retirement
    ok = _fn(".LBB0_1:\n\tds_write_b32 v3, v4\n\ts_cbranch_scc1 .LBB0_1\n")
    bad = _fn(".LBB0_1:\n\tds_write_b32 v3, v4\n\tds_read_b32 v5, v3\n\ts_cbranch_scc1 .LBB0_1\n")
    assert check_isa.check_text(ok) == []
    assert check_isa.check_text(bad) != []
    counted = _fn("\tds_read_b128 v[80:83], v84\n\tds_write_b32 v3, v4\n\ts_waitcnt lgkmcnt(1)\n"
                  "\tv_mov_b32_e32 v1, v81\n")
    assert check_isa.check_text(counted) == []
