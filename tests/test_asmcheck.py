"""The post-build wait check (asmcheck): planted hazards in small disassembly listings are found,
correct waits pass, and every object of the built library is free of them."""

from __future__ import annotations

from pathlib import Path

import pytest

from ivonar_amd import asmcheck

BUILD = Path(__file__).resolve().parent.parent / "ivonar-inference_amd" / "_build"


def _listing(body) -> str:
    """A function in llvm-objdump's layout: label, then one instruction per line with its address and,
    for a branch (given as (text, target index)), the target in the trailing comment."""
    lines = ["0000000000001000 <kernel>:"]
    for i, item in enumerate(body):
        text, target = item if isinstance(item, tuple) else (item, None)
        note = f" <kernel+0x{8 * target:x}>" if target is not None else ""
        lines.append(f"\t{text:<58}// {0x1000 + 8 * i:012X}: 00000000{note}")
    return "\n".join(lines)


def _branch(text: str, target_index: int):
    return (text, target_index)


def _hazards(body) -> list[asmcheck.Hazard]:
    (fn,) = asmcheck.parse_disassembly(_listing(body))
    return asmcheck.check_function(fn)


def test_read_before_the_covering_wait_is_found():
    body = [
        "global_load_dwordx4 v[4:7], v[0:1], off",
        "global_load_dword v8, v[2:3], off",
        "s_waitcnt vmcnt(1)",  # the dwordx4 has landed, v8 has not
        "v_add_u32_e32 v9, v4, v7",
        "v_mov_b32_e32 v10, v8",  # planted: v8 still in flight
        "s_waitcnt vmcnt(0)",
        "v_mov_b32_e32 v11, v8",
        "s_endpgm",
    ]
    hazards = _hazards(body)
    assert [h.registers for h in hazards] == [[8]]
    assert "v_mov_b32_e32 v10, v8" in hazards[0].text


def test_correct_waits_pass_and_stores_count():
    body = [
        "global_load_dword v8, v[2:3], off",
        "global_store_dword v[0:1], v5, off",
        "global_load_dword v9, v[2:3], off",
        "s_waitcnt vmcnt(2)",  # v8 has two younger vector memory ops: landed
        "v_mov_b32_e32 v10, v8",
        "s_waitcnt vmcnt(0)",
        "v_mov_b32_e32 v11, v9",
        "s_endpgm",
    ]
    assert _hazards(body) == []
    body[3] = "s_waitcnt vmcnt(3)"  # too weak: v8 may still be in flight
    assert [h.registers for h in _hazards(body)] == [[8]]


def test_value_carried_across_a_loop_back_edge_is_found():
    # The shape of the defect in the long-row GEMV: a side load issued in one iteration is copied at the
    # top of the next before the wait that covers it.
    body = [
        "global_load_dword v20, v[2:3], off",       # 0: side load of the first item
        "s_waitcnt vmcnt(0)",                        # 1
        "v_mov_b32_e32 v21, v20",                    # 2: loop top, copy of the carried side value
        "global_load_dwordx4 v[4:7], v[0:1], off",  # 3: refill
        "global_load_dword v20, v[2:3], off",       # 4: next item's side load
        "s_waitcnt vmcnt(1)",                        # 5: covers the refill only
        "v_add_u32_e32 v8, v4, v21",                 # 6
        _branch("s_cbranch_scc1 65530", 2),          # 7: back to the loop top
        "s_waitcnt vmcnt(0)",                        # 8
        "s_endpgm",                                  # 9
    ]
    hazards = _hazards(body)
    assert [(h.address, h.registers) for h in hazards] == [(16, [20])]
    body[5] = "s_waitcnt vmcnt(0)"
    assert _hazards(body) == []


def test_pending_on_one_path_counts_at_the_join():
    body = [
        _branch("s_cbranch_execz 3", 3),             # 0: skip the load
        "global_load_dword v8, v[2:3], off",         # 1
        "s_nop 0",                                   # 2
        "v_mov_b32_e32 v9, v8",                      # 3: join; v8 pending on the fall-through path
        "s_endpgm",
    ]
    assert [h.registers for h in _hazards(body)] == [[8]]


def test_lds_dma_and_load_over_load_are_not_reported():
    body = [
        "buffer_load_dword v1, s[8:11], 0 offen lds",
        "global_load_dword v8, v[2:3], off",
        "global_load_dword v8, v[4:5], off",
        "s_waitcnt vmcnt(0)",
        "v_mov_b32_e32 v9, v8",
        "s_endpgm",
    ]
    assert _hazards(body) == []


@pytest.mark.skipif(not any(BUILD.glob("*.o")), reason="the HIP library has not been built here")
def test_built_objects_have_no_early_reads():
    hazards = [h for obj in sorted(BUILD.glob("*.o")) for h in asmcheck.check_object(obj)]
    assert not hazards, "\n".join(map(str, hazards[:10]))


@pytest.mark.skipif(not any(BUILD.glob("*.o")), reason="the HIP library has not been built here")
def test_built_kernels_use_no_scratch():
    spills = [entry for obj in sorted(BUILD.glob("*.o")) for entry in asmcheck.kernels_with_scratch(obj)]
    assert not spills, spills[:10]
