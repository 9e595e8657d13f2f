"""Checks on the gfx950 assembly the compiler makes of the HIP sources (CPU only:
hipcc cross-compiles).

* No FLAT memory instruction.  Every device-buffer access goes through a
  global-address-space pointer; a FLAT store counts in lgkmcnt as well as
  vmcnt, so each later wait for an LDS access would also wait for it to reach
  memory.
* No dropped VCC -> SCC copy.  A wave-uniform condition that the compiler forms
  with a vector compare (64-bit compares have no scalar form) and then uses both
  for a branch on VCC and for an s_cselect needs an `s_and_b64 vcc, vcc, exec`
  in between.  The compiler's exec-mask peephole has removed that copy: the
  select then read a stale SCC (the ragged-K kernel wrote every row of a split
  output to the second tensor).  The pattern looked for is a VCC-writing
  v_cmp, then an SCC reader with no SCC writer in between, before the branch
  on that VCC.
"""

import concurrent.futures as cf
import re
import shutil
import subprocess
from pathlib import Path

import pytest

from nanopysche_amd import build as B

HIP_SOURCES = [s for s in B.SOURCES if s.endswith(".hip")]

SCC_WRITE = re.compile(r"^s_(cmp|cmpk|and|or|xor|andn2|orn2|nand|nor|xnor|add_|sub_|addc|subb|lshl|lshr|ashr|bfe|"
                       r"min|max|abs|not|bcnt|absdiff|bitcmp|mul_hi)")
SCC_READ = re.compile(r"^(s_cselect|s_cbranch_scc|s_cmov)")
VCC_CMP = re.compile(r"^v_cmp\w*(_e32\s+vcc|_e64\s+vcc,)")
VCC_WRITE = re.compile(r"^(v_cmp\w*(_e32\s+vcc|_e64\s+vcc,)|s_\w+ vcc,|v_\w+ vcc,|s_mov_b64 vcc)")
KERNEL = re.compile(r"^(_Z\w+):")


def dropped_scc_copies(asm: str):
    """(line, kernel) of each branch on VCC whose compare fed an SCC reader with
    no SCC writer after the compare."""
    lines = [ln.strip() for ln in asm.split("\n")]
    found, kern = [], None
    for i, t in enumerate(lines):
        m = KERNEL.match(t)
        if m:
            kern = m.group(1)
            continue
        if not re.match(r"^s_cbranch_vccn?z", t):
            continue
        reader = False
        for j in range(i - 1, max(i - 80, 0), -1):
            u = lines[j]
            if KERNEL.match(u):
                break
            if not u or u[0] in ";.":
                continue
            if VCC_WRITE.match(u):
                if VCC_CMP.match(u) and reader:
                    found.append((i + 1, kern))
                break
            if SCC_WRITE.match(u):
                reader = False
            elif SCC_READ.match(u):
                reader = True
    return found


def test_checker_finds_the_dropped_copy():
    """The pattern check on a hand-written fragment: with the copy, and without."""
    good = """_ZN2fm1kE:
\tv_cmp_gt_i64_e32 vcc, s[6:7], v[180:181]
\ts_and_b64 vcc, vcc, exec
\ts_cselect_b32 s6, s75, 0x24508
\ts_cbranch_vccnz .LBB0_1
"""
    bad = good.replace("\ts_and_b64 vcc, vcc, exec\n", "")
    assert dropped_scc_copies(good) == []
    assert dropped_scc_copies(bad) == [(4, "_ZN2fm1kE")]


@pytest.fixture(scope="module")
def device_asm(tmp_path_factory):
    if shutil.which("hipcc") is None and not Path("/opt/rocm/bin/hipcc").exists():
        pytest.skip("hipcc not available")
    out = tmp_path_factory.mktemp("isa")

    def compile_one(src):
        dst = out / (src + ".s")
        cmd = [B._hipcc(), *B._flags(), "--cuda-device-only", "-S", "-x", "hip", str(B.CSRC / src), "-o", str(dst)]
        r = subprocess.run(cmd, capture_output=True, text=True)
        assert r.returncode == 0, r.stderr[-2000:]
        return src, dst.read_text()

    with cf.ThreadPoolExecutor(len(HIP_SOURCES)) as ex:
        return dict(ex.map(compile_one, HIP_SOURCES))


@pytest.mark.timeout(900)
@pytest.mark.parametrize("src", HIP_SOURCES)
def test_no_flat_memory_instructions(device_asm, src):
    flat = [ln.strip() for ln in device_asm[src].split("\n") if re.match(r"^\s+flat_(load|store|atomic)", ln)]
    assert flat == [], f"{src}: {len(flat)} FLAT instructions, first {flat[:3]}"


@pytest.mark.timeout(900)
@pytest.mark.parametrize("src", HIP_SOURCES)
def test_no_dropped_vcc_to_scc_copy(device_asm, src):
    found = dropped_scc_copies(device_asm[src])
    assert found == [], f"{src}: {found[:5]}"
