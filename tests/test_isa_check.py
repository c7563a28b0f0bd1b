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
    """Lines starting with "asm " are wrapped in the compiler's inline-asm markers."""
    out = []
    for l in body:
        if l.endswith(":"):
            out.append(l)
        elif l.startswith("asm "):
            out += ["\t;;#ASMSTART", "\t" + l[4:], "\t;;#ASMEND"]
        else:
            out.append("\t" + l)
    return "_Zkernel:\n" + "\n".join(out) + "\n.Lfunc_end0:\n"


def _bad(body):
    return [t for v in ic.check_asm(_fn(body)).values() for _, t in v]


def test_copy_before_wait_is_reported():
    body = ["asm ds_read2st64_b32 v[4:5], v1 offset0:0 offset1:1",
            "v_mov_b32_e32 v8, v4",          # planted: copies a register still being filled
            "s_waitcnt lgkmcnt(0)",
            "v_fmac_f32_e32 v9, v8, v5",
            "s_endpgm"]
    assert _bad(body) == ["v_mov_b32_e32 v8, v4"]
    fixed = [body[0], body[2], body[1], body[3], body[4]]
    assert _bad(fixed) == []


def test_in_order_retirement():
    body = ["asm ds_read_b128 v[0:3], v10",
            "asm ds_read_b128 v[4:7], v11",
            "s_waitcnt lgkmcnt(1)",         # the first read has landed, the second may not
            "v_add_f32_e32 v20, v0, v1",
            "v_add_f32_e32 v21, v4, v5",    # planted
            "s_endpgm"]
    assert _bad(body) == ["v_add_f32_e32 v21, v4, v5"]


def test_overwrite_and_address_in_flight():
    body = ["asm ds_read_b64 v[2:3], v1",
            "v_mov_b32_e32 v3, 0",          # planted: overwrites a register still being filled
            "ds_read_b32 v6, v2",           # planted: address register in flight
            "s_waitcnt lgkmcnt(0)",
            "s_endpgm"]
    assert sorted(_bad(body)) == ["ds_read_b32 v6, v2", "v_mov_b32_e32 v3, 0"]


def test_across_branches_and_loops():
    body = ["asm ds_read_b32 v2, v1",
            "s_cbranch_scc0 .LBB0_2",
            "s_waitcnt lgkmcnt(0)",
            ".LBB0_2:",
            "v_mov_b32_e32 v3, v2",         # planted: reached without the wait on the taken path
            "s_endpgm"]
    assert _bad(body) == ["v_mov_b32_e32 v3, v2"]
    loop = [".LBB0_1:",
            "v_add_f32_e32 v4, v4, v2",     # planted: the read of the previous iteration
            "asm ds_read_b32 v2, v1",
            "s_cbranch_scc1 .LBB0_1",
            "s_waitcnt lgkmcnt(0)",
            "s_endpgm"]
    # the read itself is reported too: its destination is still being filled
    # by the previous iteration's read
    assert sorted(_bad(loop)) == ["ds_read_b32 v2, v1", "v_add_f32_e32 v4, v4, v2"]
    loop_ok = [".LBB0_1:", "asm ds_read_b32 v2, v1", "s_waitcnt lgkmcnt(0)",
               "v_add_f32_e32 v4, v4, v2", "s_cbranch_scc1 .LBB0_1", "s_endpgm"]
    assert _bad(loop_ok) == []


def test_vector_memory_loads():
    """Loads from inline asm (Q in the flash kernels) are waited for with vmcnt:
    every vector load, the compiler's and the LDS-DMA copies included, takes
    a place in the order, and only the asm loads' registers are tracked."""
    body = ["asm global_load_dwordx4 v[0:3], v[8:9], off",      # Q
            "global_load_lds_dwordx4 v[10:11], off",             # tile copies
            "global_load_lds_dwordx4 v[12:13], off",
            "s_waitcnt vmcnt(2)",                                # Q has landed
            "v_mov_b32_e32 v20, v0",
            "s_endpgm"]
    assert _bad(body) == []
    early = list(body)
    early[3] = "s_waitcnt vmcnt(3)"                              # planted: Q may be in flight
    assert _bad(early) == ["v_mov_b32_e32 v20, v0"]
    tracked = ["global_load_dwordx4 v[0:3], v[8:9], off",       # the compiler's own load
               "v_mov_b32_e32 v20, v0", "s_endpgm"]
    assert _bad(tracked) == []


def test_compiler_reads_count_but_are_not_tracked():
    body = ["asm ds_read_b128 v[0:3], v10",
            "ds_read_b128 v[4:7], v11",                          # the compiler's own read
            "s_waitcnt lgkmcnt(1)",                              # the asm read has landed
            "v_mov_b32_e32 v20, v0",
            "v_mov_b32_e32 v21, v4",                             # the compiler waits for its own
            "s_endpgm"]
    assert _bad(body) == []


def test_library_sources_are_checked_by_the_build():
    """build.py runs the check on every .hip source; the built library exists
    only if all of them passed (it raises otherwise)."""
    src = open(os.path.join(HERE, "..", "jules_amd", "build.py")).read()
    assert "_check_lds_waits(src, path, lang, verbose)" in src
    if not os.path.exists(os.path.join(HERE, "..", "jules_amd", "libjules_hip.so")):
        pytest.skip("library not built")
