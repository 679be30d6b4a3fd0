"""The build-time check of inline-asm load registers (flashgrpo_amd._isa_check) on small
hand-written kernels shaped like the LM head's weight stream: loads into registers, an
LDS-DMA load, a loop whose reissued loads are waited for at its head, and the mistakes
the check exists to catch (a copy, a spill or a use of a register whose load may still be
in flight, on any path)."""
import sys
import os

sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "ss-grpo_amd"))

from flashgrpo_amd._isa_check import check_asm  # noqa: E402

HEAD = "_Zkernel:\n"
TAIL = "\ts_endpgm\n.Lfunc_end0:\n"


def kernel(body: str) -> str:
    return HEAD + body + TAIL


def hazards(body: str):
    n, hz = check_asm(kernel(body))
    assert n == 1
    return hz


STREAM = """
\tbuffer_load_dwordx4 v[10:13], v1, s[4:7], s8 offen
\tbuffer_load_dwordx4 v[14:17], v1, s[4:7], s9 offen
{pre}
.LBB0_1:
\ts_waitcnt vmcnt(1)
\ts_barrier
{head}
\tds_write_b128 v20, v[10:13]
{mid}
\tbuffer_load_dwordx4 v2, s[4:7], s8 offen lds
\tbuffer_load_dwordx4 v[10:13], v1, s[4:7], s9 offen
\ts_waitcnt vmcnt(2)
\tds_write_b128 v21, v[14:17]
\tbuffer_load_dwordx4 v[14:17], v1, s[4:7], s9 offen
{tail}
\ts_cbranch_scc1 .LBB0_1
\ts_waitcnt vmcnt(0)
\tv_mov_b32 v10, 0
"""


def stream(pre="", head="", mid="", tail=""):
    return STREAM.format(pre=pre, head=head, mid=mid, tail=tail)


def test_clean_stream_passes():
    assert hazards(stream()) == []


def test_copy_right_after_a_load_is_caught():
    hz = hazards(stream(pre="\tv_mov_b32 v30, v11"))
    assert len(hz) == 1 and hz[0][3] == [("v", 11)]


def test_use_of_the_other_slot_in_the_loop_is_caught():
    # v[14:17] is younger than the load the head's vmcnt(1) waits for
    hz = hazards(stream(head="\tv_mov_b32 v30, v15"))
    assert [h[3] for h in hz] == [[("v", 15)]]


def test_loaded_slot_is_free_after_its_wait():
    assert hazards(stream(head="\tv_mov_b32 v30, v12")) == []


def test_spill_of_an_in_flight_register_is_caught():
    hz = hazards(stream(mid="\tscratch_store_dwordx4 off, v[10:13], off offset:16"))
    assert hz == []  # v[10:13] landed at the head's wait, before the reissue
    hz = hazards(stream(tail="\tscratch_store_dwordx4 off, v[10:13], off offset:16"))
    assert len(hz) == 1 and hz[0][3][0] == ("v", 10)


def test_reissued_loads_reach_the_loop_head_through_the_back_edge():
    # nothing is in flight on the first entry; before the head's wait, the loads issued at
    # the end of the previous iteration may be
    body = stream(pre="\ts_waitcnt vmcnt(0)").replace(".LBB0_1:\n", ".LBB0_1:\n\tv_mov_b32 v30, v14\n")
    hz = hazards(body)
    assert len(hz) == 1 and hz[0][3] == [("v", 14)]
    assert hazards(stream(pre="\ts_waitcnt vmcnt(0)")) == []


def test_branch_that_skips_the_wait_is_caught():
    body = """
\tbuffer_load_dwordx4 v[10:13], v1, s[4:7], s8 offen
\ts_cbranch_vccz .LBB0_2
\ts_waitcnt vmcnt(0)
.LBB0_2:
\tv_add_u32_e32 v30, v10, v31
"""
    hz = hazards(body)
    assert len(hz) == 1 and hz[0][3] == [("v", 10)]
    assert hazards(body.replace("\ts_cbranch_vccz .LBB0_2\n", "")) == []


def test_lds_dma_and_stores_count_but_write_no_registers():
    body = """
\tbuffer_load_dwordx4 v[10:13], v1, s[4:7], s8 offen
\tbuffer_load_dwordx4 v2, s[4:7], s8 offen lds
\tglobal_store_dwordx2 v[40:41], v[42:43], off
\ts_waitcnt vmcnt(2)
\tv_mov_b32 v30, v10
\tv_mov_b32 v31, v2
"""
    assert hazards(body) == []
    assert hazards(body.replace("vmcnt(2)", "vmcnt(3)")) != []
