"""Static checks of every kernel's device assembly, built with the library's
own flags (make asm): no register of an LDS read is used before the wait that
covers it (kvbridge_amd/csrc/check_lds_waits.py), and every hand-counted
vector-memory wait leaves no load of an older tile DMA group in flight
(kvbridge_amd/csrc/check_vm_waits.py), with planted mistakes that each check
must catch."""
import os
import subprocess
import sys
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "kvbridge_amd", "csrc")
sys.path.insert(0, CSRC)
import check_lds_waits as C  # noqa: E402
import check_vm_waits as V  # noqa: E402


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


@pytest.fixture(scope="module")
def asm_files(tmp_path_factory):
    """Device assembly of every kernel file, built with the library's flags."""
    tmp = str(tmp_path_factory.mktemp("asm"))
    r = subprocess.run(["make", "-s", "-j8", "-C", CSRC, "asm", f"BUILD={tmp}"], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    files = sorted(os.path.join(tmp, "asm", f) for f in os.listdir(os.path.join(tmp, "asm")) if f.endswith(".s"))
    assert len(files) >= 8
    return {os.path.basename(f): open(f).read() for f in files}


@pytest.mark.timeout(900)
def test_every_kernel_waits_before_using_lds_reads(asm_files):
    findings = {f: C.scan_asm(text) for f, text in asm_files.items()}
    bad = {f: {n: v[:2] for n, v in d.items()} for f, d in findings.items() if d}
    assert not bad, bad


# ---- hand-counted vector-memory waits (check_vm_waits.py) -------------------

_PC_LOOP = """_Zpc:
	s_load_dword s2, s[0:1], 0x0
{g}
{g}
.LBB0_1:
	s_cbranch_scc1 .LBB0_2
	;;#ASMSTART
	s_waitcnt vmcnt({n}) ; kvb-keep 1
	;;#ASMEND
.LBB0_2:
	s_barrier
	s_cbranch_scc1 .LBB0_3
{g}
.LBB0_3:
	s_cbranch_scc0 .LBB0_1
	s_endpgm
.Lfunc_end0:
"""


def _group(k):
    return "\t;;#ASMSTART\n\t;kvb-dma-group\n\t;;#ASMEND\n" + "\tglobal_load_lds_dwordx4 v[4:5], off nt\n" * k


def test_vm_checker_accepts_exact_groups():
    # Two tiles in flight, three loads each, wait for all but the newest three:
    # also on the loop's last steps, where no new tile is issued.
    f, n, sizes = V.scan_asm(_PC_LOOP.format(g=_group(3), n=3))["_Zpc"]
    assert f == [] and n == 1 and sizes == {3}


def test_vm_checker_flags_short_groups():
    # The toolchain emits two loads per tile where the wait assumes three: the
    # wait leaves a load of the older tile in flight.
    f, n, sizes = V.scan_asm(_PC_LOOP.format(g=_group(2), n=3))["_Zpc"]
    assert n == 1 and sizes == {2} and len(f) == 1 and "older" in f[0][2]


def test_vm_checker_counts_stores_and_rejects_unannotated_waits():
    # Any vector-memory operation after the older tile counts toward N (a
    # store here); a hand-written vmcnt(N > 0) without kvb-keep is reported.
    text = _PC_LOOP.format(g=_group(2) + "\tglobal_store_dword v[0:1], v2, off\n", n=3)
    assert V.scan_asm(text)["_Zpc"][0] == []
    text = text.replace(" ; kvb-keep 1", "")
    f = V.scan_asm(text)["_Zpc"][0]
    assert f and "annotation" in f[0][2]


def _drop_last_dma_per_block(text):
    """Planted mistake: every basic block that issues LDS-DMA loads emits one
    fewer (a toolchain that drops an instruction of each tile)."""
    lines = text.split("\n")
    last, drop = None, set()
    for i, line in enumerate(lines):
        t = line.split(";")[0].strip()
        if V._LABEL.match(t) or V._TARGET.match(t) or t.startswith("s_endpgm"):
            if last is not None:
                drop.add(last)
            last = None
        elif V._is_dma(t):
            last = i
    if last is not None:
        drop.add(last)
    return "\n".join(x for i, x in enumerate(lines) if i not in drop)


@pytest.mark.timeout(900)
def test_hand_counted_vm_waits_hold_and_planted_short_tiles_are_caught(asm_files):
    checked = {}
    for f, text in asm_files.items():
        for name, (found, n, sizes) in V.scan_asm(text).items():
            assert not found, (f, name, found[:2])
            checked[name] = (n, sizes)
    # The dense-geometry kernel's DMA wave: one hand-counted wait, 34 loads
    # per tile (split_i8_rows.hip kLoadsPerTile).
    pc = {n: v for n, v in checked.items() if "split_i8_rows_pc_kernel" in n}
    assert len(pc) == 2 and all(v == (1, {34}) for v in pc.values()), pc
    lds = {n: v for n, v in checked.items() if "split_lds_kernel" in n and v[0] > 0}
    assert len(lds) >= 8, lds
    # One load fewer per tile must be caught in every kernel whose waits
    # depend on the count (the dense kernel and the f16 LDS kernels).
    for f in ("split_i8_rows.s", "split_lds.s"):
        planted = V.scan_asm(_drop_last_dma_per_block(asm_files[f]))
        for name, (found, n, _) in planted.items():
            if n and ("split_i8_rows_pc_kernel" in name or "split_lds_kernel" in name):
                assert found, f"{name}: planted short tiles not caught"
