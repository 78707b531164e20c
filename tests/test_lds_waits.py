"""Static check of every kernel's device assembly (kvbridge_amd/csrc/
check_lds_waits.py): no register of an LDS read is used before the wait that
covers it.  Builds the assembly with the library's own flags (make asm)."""
import os
import subprocess
import sys
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "kvbridge_amd", "csrc")
sys.path.insert(0, CSRC)
import check_lds_waits as C  # noqa: E402


def test_scanner_flags_a_use_before_the_wait():
    asm = """_Zfoo:
\tds_read_b128 v[4:7], v1 offset:16
\tds_read_b128 v[8:11], v1 offset:32
\ts_waitcnt lgkmcnt(1)
\tv_mov_b32_e32 v20, v4
\tv_accvgpr_write_b32 a3, v9
\ts_waitcnt lgkmcnt(0)
\tv_mov_b32_e32 v21, v10
.Lfunc_end0:
"""
    found = C.scan_asm(asm)["_Zfoo"]
    assert [t for _, t in found] == ["v_accvgpr_write_b32 a3, v9"]  # v4 was covered by lgkmcnt(1)


def test_scanner_accepts_waited_reads_and_other_lgkm_ops():
    asm = """_Zbar:
\ts_load_dword s2, s[0:1], 0x0
\tds_read_b32 v3, v1
\ts_waitcnt lgkmcnt(0)
\tv_add_u32_e32 v4, v3, v3
\tds_read_b32 v5, v1 offset:4
\tv_add_u32_e32 v6, v7, v8
\ts_waitcnt lgkmcnt(0)
\tv_add_u32_e32 v6, v5, v5
.Lfunc_end1:
"""
    assert C.scan_asm(asm) == {}


def test_scanner_follows_branches():
    """A read pending in an out-of-line block reaches only that block's
    successors: the block after its unconditional branch in file order is
    not one, its branch target is."""
    asm = """_Zcfg:
\ts_cbranch_vccz .LBB0_3
\ts_cbranch_scc1 .LBB0_2
\ts_endpgm
.LBB0_2:
\tds_read_b128 v[8:11], v1
\ts_branch .LBB0_4
.LBB0_3:
\tv_mov_b32_e32 v22, v8
\ts_endpgm
.LBB0_4:
\tv_mov_b32_e32 v23, v9
\ts_waitcnt lgkmcnt(0)
\tv_mov_b32_e32 v24, v10
\ts_endpgm
.Lfunc_end2:
"""
    found = C.scan_asm(asm)["_Zcfg"]
    assert [t for _, t in found] == ["v_mov_b32_e32 v23, v9"]


@pytest.mark.timeout(900)
def test_every_kernel_waits_before_using_lds_reads():
    with tempfile.TemporaryDirectory() as tmp:
        r = subprocess.run(["make", "-s", "-j8", "-C", CSRC, "asm", f"BUILD={tmp}"], capture_output=True, text=True)
        assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
        files = sorted(os.path.join(tmp, "asm", f) for f in os.listdir(os.path.join(tmp, "asm")) if f.endswith(".s"))
        assert len(files) >= 8
        findings = {f: C.scan_asm(open(f).read()) for f in files}
    bad = {os.path.basename(f): {n: v[:2] for n, v in d.items()} for f, d in findings.items() if d}
    assert not bad, bad
