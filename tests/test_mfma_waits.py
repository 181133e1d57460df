"""Reads of MFMA results in this library's gfx950 assembly wait ten states on
every path (symmetrix-xl_amd/csrc/check_mfma_waits.py).

A read that comes too early returns a stale accumulator element with no
error.  The compiler has padded only the fall-through path into a join: the
edge-MLP reverse read its last accumulator register right after its MFMA on
the taken branch, and radial-adjoint columns 3 and 7 came out wrong.  The
checker's own logic is tested on planted listings; the library's kernels are
checked on their generated assembly (make check-waits).
"""

import os
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "symmetrix-xl_amd", "csrc")
sys.path.insert(0, CSRC)
import check_mfma_waits as cw  # noqa: E402

# the shape of the failure: the accumulator is zeroed, a branch skips the MFMA, the join reads it
TAKEN_BRANCH = """_Zk:
\tv_accvgpr_write_b32 a3, 0
\ts_cbranch_vccnz .LBB0_2
\tv_mfma_f32_16x16x4_f32 a[0:3], v7, v24, a[0:3]
.LBB0_2:
\tv_accvgpr_read_b32 v4, a3
\ts_nop 7
\tv_accvgpr_read_b32 v7, a1
\tglobal_store_dword v[0:1], v4, off
\ts_endpgm
"""

# the same join with the chain settled inside its block (sixteen wait states)
SETTLED = """_Zk:
\tv_accvgpr_write_b32 a3, 0
\ts_cbranch_vccnz .LBB0_2
\tv_mfma_f32_16x16x4_f32 a[0:3], v7, v24, a[0:3]
\ts_nop 7
\ts_nop 7
.LBB0_2:
\tv_accvgpr_read_b32 v4, a3
\tv_accvgpr_read_b32 v7, a1
\ts_endpgm
"""

# a store of an MFMA result on the branch path; the fall-through path is padded
STORE_ON_BRANCH = """_Zk:
\tv_mfma_f32_16x16x4_f32 v[8:11], v1, v2, 0
\ts_cbranch_scc1 .LBB0_3
\ts_nop 9
\tv_add_f32_e32 v3, v8, v3
.LBB0_3:
\tglobal_store_dwordx4 v[4:5], v[8:11], off
\ts_endpgm
"""


def _check(text):
    (name, body), = cw.split_kernels(text.split("\n"))
    return cw.findings(body, 10)


def test_planted_early_reads_are_found():
    got = _check(TAKEN_BRANCH)
    assert [(ins.split()[0], reg, d) for _, ins, reg, d in got] == [
        ("v_accvgpr_read_b32", "a3", 0), ("v_accvgpr_read_b32", "a1", 9)]
    got = _check(STORE_ON_BRANCH)
    assert {(reg, d) for _, _, reg, d in got} == {("v8", 1), ("v9", 1), ("v10", 1), ("v11", 1)}


def test_settled_chains_pass():
    assert _check(SETTLED) == []


@pytest.mark.skipif(shutil.which("make") is None or not os.path.exists("/opt/rocm/bin/hipcc"),
                    reason="needs hipcc to generate the assembly")
def test_library_kernels_read_mfma_results_late_enough():
    res = subprocess.run(["make", "-C", CSRC, "-j2", "check-waits"], capture_output=True, text=True, timeout=1500)
    assert res.returncode == 0, res.stdout[-3000:] + res.stderr[-3000:]
    assert "functions checked" in res.stdout
