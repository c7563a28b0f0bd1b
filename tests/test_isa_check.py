"""The build's static check of asm-issued LDS reads (jules_amd/isa_check.py),
on hand-written gfx950 assembly with planted mistakes: each planted use of
a register before the wait that covers its LDS read must be reported, and
the same code with the wait in place must pass."""
import importlib.util
import os

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
_spec = importlib.util.spec_from_file_location(
    "jules_isa_check", os.path.join(HERE, "..", "jules_amd", "isa_check.py"))
ic = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(ic)


def _fn(body):
    return "_Zkernel:\n" + "\n".join("\t" + l if not l.endswith(":") else l for l in body) + \
        "\n.Lfunc_end0:\n"


def _bad(body):
    return [t for v in ic.check_asm(_fn(body)).values() for _, t in v]


def test_copy_before_wait_is_reported():
    body = ["ds_read2st64_b32 v[4:5], v1 offset0:0 offset1:1",
            "v_mov_b32_e32 v8, v4",          # planted: copies a register still being filled
            "s_waitcnt lgkmcnt(0)",
            "v_fmac_f32_e32 v9, v8, v5",
            "s_endpgm"]
    assert _bad(body) == ["v_mov_b32_e32 v8, v4"]
    fixed = [body[0], body[2], body[1], body[3], body[4]]
    assert _bad(fixed) == []


def test_in_order_retirement():
    body = ["ds_read_b128 v[0:3], v10",
            "ds_read_b128 v[4:7], v11",
            "s_waitcnt lgkmcnt(1)",         # the first read has landed, the second may not
            "v_add_f32_e32 v20, v0, v1",
            "v_add_f32_e32 v21, v4, v5",    # planted
            "s_endpgm"]
    assert _bad(body) == ["v_add_f32_e32 v21, v4, v5"]


def test_overwrite_and_address_in_flight():
    body = ["ds_read_b64 v[2:3], v1",
            "v_mov_b32_e32 v3, 0",          # planted: overwrites a register still being filled
            "ds_read_b32 v6, v2",           # planted: address register in flight
            "s_waitcnt lgkmcnt(0)",
            "s_endpgm"]
    assert sorted(_bad(body)) == ["ds_read_b32 v6, v2", "v_mov_b32_e32 v3, 0"]


def test_across_branches_and_loops():
    body = ["ds_read_b32 v2, v1",
            "s_cbranch_scc0 .LBB0_2",
            "s_waitcnt lgkmcnt(0)",
            ".LBB0_2:",
            "v_mov_b32_e32 v3, v2",         # planted: reached without the wait on the taken path
            "s_endpgm"]
    assert _bad(body) == ["v_mov_b32_e32 v3, v2"]
    loop = [".LBB0_1:",
            "v_add_f32_e32 v4, v4, v2",     # planted: the read of the previous iteration
            "ds_read_b32 v2, v1",
            "s_cbranch_scc1 .LBB0_1",
            "s_waitcnt lgkmcnt(0)",
            "s_endpgm"]
    # the read itself is reported too: its destination is still being filled
    # by the previous iteration's read
    assert sorted(_bad(loop)) == ["ds_read_b32 v2, v1", "v_add_f32_e32 v4, v4, v2"]
    loop_ok = [".LBB0_1:", "ds_read_b32 v2, v1", "s_waitcnt lgkmcnt(0)",
               "v_add_f32_e32 v4, v4, v2", "s_cbranch_scc1 .LBB0_1", "s_endpgm"]
    assert _bad(loop_ok) == []


def test_library_sources_are_checked_by_the_build():
    """build.py runs the check on every .hip source; the built library exists
    only if all of them passed (it raises otherwise)."""
    src = open(os.path.join(HERE, "..", "jules_amd", "build.py")).read()
    assert "_check_lds_waits(src, path, lang, verbose)" in src
    if not os.path.exists(os.path.join(HERE, "..", "jules_amd", "libjules_hip.so")):
        pytest.skip("library not built")
