"""The static check of hand-counted LDS waits (qtpytorch_amd/csrc/check_lgkm.py)
on synthetic assembly with planted mistakes, and on the GEMM source itself."""
import os
import shutil

import pytest

from qtpytorch_amd.csrc import check_lgkm as ck

HEAD = "_Z4kernv:\n"
TAIL = "\ts_endpgm\n.Lfunc_end0:\n"


def asm_read(op, dst, off=0):
    return f"\t;;#ASMSTART\n\t{op} {dst}, v100 offset:{off}\n\t;;#ASMEND\n"


def asm_wait(n):
    return f"\t;;#ASMSTART\n\ts_waitcnt lgkmcnt({n})\n\t;;#ASMEND\n"


def run(body):
    n, problems = ck.check_asm(HEAD + body + TAIL)
    assert n == 1
    return problems


def test_wait_then_use_is_clean():
    body = asm_read("ds_read_b128", "v[0:3]") + asm_wait(0) + "\tv_add_f32_e32 v10, v0, v1\n"
    assert run(body) == []


def test_use_before_wait_is_reported():
    body = asm_read("ds_read_b128", "v[0:3]") + "\tv_add_f32_e32 v10, v2, v1\n" + asm_wait(0)
    assert len(run(body)) == 1


def test_overwrite_before_wait_is_reported():
    # the read's data would land on top of the compiler's new value
    body = asm_read("ds_read_b128", "v[0:3]") + "\tv_mov_b32_e32 v3, 0\n" + asm_wait(0)
    assert len(run(body)) == 1


def test_counts_retire_in_issue_order():
    two = asm_read("ds_read_b128", "v[0:3]") + asm_read("ds_read_b128", "v[4:7]", 16) + asm_wait(1)
    assert run(two + "\tv_add_f32_e32 v10, v0, v1\n") == []           # the first read retired
    assert len(run(two + "\tv_add_f32_e32 v10, v4, v1\n")) == 1       # the second may still be in flight


def test_scalar_loads_do_not_count_toward_the_wait():
    # a scalar load can complete before an older LDS read, so with one of
    # each outstanding lgkmcnt(1) does not guarantee the LDS read, whichever
    # was issued first
    for body in (asm_read("ds_read_b128", "v[0:3]") + "\ts_load_dword s4, s[0:1], 0x0\n",
                 "\ts_load_dword s4, s[0:1], 0x0\n" + asm_read("ds_read_b128", "v[0:3]")):
        assert len(run(body + asm_wait(1) + "\tv_add_f32_e32 v10, v0, v1\n")) == 1
        assert run(body + asm_wait(0) + "\tv_add_f32_e32 v10, v0, v1\n") == []


def test_transposed_read_tracked():
    body = asm_read("ds_read_b64_tr_b8", "v[8:9]") + "\tv_mov_b32_e32 v20, v9\n" + asm_wait(0)
    assert len(run(body)) == 1


def test_compiler_reads_only_count():
    # a read the compiler issued (outside inline asm) is not reported, but counts toward the queue
    body = ("\tds_read_b128 v[20:23], v100\n" + asm_read("ds_read_b128", "v[0:3]") + asm_wait(1)
            + "\tv_add_f32_e32 v10, v0, v1\n")
    assert len(run(body)) == 1


def test_loop_with_read_outstanding_at_back_edge():
    body = (".LBB0_1:\n" + asm_read("ds_read_b128", "v[0:3]") + "\ts_cbranch_scc1 .LBB0_1\n" + asm_wait(0))
    problems = run(body)
    assert any("different outstanding" in p for p in problems)


def test_loop_that_waits_each_iteration_is_clean():
    body = (".LBB0_1:\n" + asm_read("ds_read_b128", "v[0:3]") + asm_wait(0) + "\tv_add_f32_e32 v10, v0, v1\n"
            + "\ts_cbranch_scc1 .LBB0_1\n")
    assert run(body) == []


@pytest.mark.skipif(shutil.which("hipcc") is None and not os.path.exists("/opt/rocm/bin/hipcc"),
                    reason="needs hipcc")
def test_gemm_source_passes():
    from qtpytorch_amd.csrc import build as b

    src = os.path.join(os.path.dirname(ck.__file__), "mxk_gemm.hip")
    n, problems = ck.check_source(src, b.hipcc(), b.HIPCC_FLAGS)
    assert n >= 8
    assert problems == []
