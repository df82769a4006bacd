"""Static check of the sparse-MLA kernel's machine code: no register spill inside the tile loop.

The tile loop keeps the KV DMA ring in flight by counting outstanding vector-memory operations
(s_waitcnt vmcnt).  A spill reload in the loop is a vector-memory load too, and the compiler waits
for it with vmcnt(0), which drains every tile in flight each iteration.  This test compiles
csrc/sparse_mla.hip to gfx950 assembly with the library's own flags and checks that the main loop
of every multi-wave instantiation has no scratch access.
"""
import re
import shutil
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "tilelang-ascend_amd"
sys.path.insert(0, str(PKG))

HIPCC = "/opt/rocm/bin/hipcc"


@pytest.fixture(scope="module")
def asm(tmp_path_factory):
    if not Path(HIPCC).exists() and shutil.which("hipcc") is None:
        pytest.skip("hipcc not available")
    import build as B

    out = tmp_path_factory.mktemp("asm") / "sparse_mla.s"
    cmd = [HIPCC, *B.COMMON_FLAGS, *B.FILE_FLAGS.get("sparse_mla.hip", []), "-S", "--cuda-device-only",
           str(PKG / "csrc" / "sparse_mla.hip"), "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True)
    return out.read_text()


def test_no_spill_in_the_tile_loop(asm):
    names = re.findall(r"^(_ZN3dsa\d+sparse_mla_(?:rows2_)?kernel\S+):", asm, re.M)
    assert len(names) >= 6, names
    checked = 0
    for name in names:
        if "ILi1E" in name:  # one wave per workgroup: only small head counts, one tile in flight anyway
            continue
        a = asm.index(name + ":")
        b = asm.index(".Lfunc_end", a)
        in_loop = False
        for line in asm[a:b].split("\n"):
            line = line.strip()
            if re.match(r"^\.LBB\S+:", line):
                in_loop = "Loop" in line
            elif in_loop:
                assert "scratch_" not in line, f"{name}: spill in the tile loop: {line}"
        checked += 1
    assert checked >= 4
