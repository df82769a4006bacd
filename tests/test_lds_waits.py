"""Static check: every explicit LDS wait in the gather and decode kernels covers the reads it guards.

csrc/sparse_mla.hip, csrc/sparse_flash_mla.hip and csrc/sparse_gqa.hip issue their LDS operand reads
as inline asm and wait for them with counted ``s_waitcnt lgkmcnt(N)``.  This test compiles the files to gfx950
assembly with the library's own flags and replays the LDS counter through each kernel's control
flow (tests/asm_lds.py): no instruction may touch a register whose LDS load may still be in
flight.  The planted case below shows the check sees an off-by-eight count.
"""
import shutil
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "tilelang-ascend_amd"
sys.path.insert(0, str(PKG))
sys.path.insert(0, str(Path(__file__).resolve().parent))

import asm_lds  # noqa: E402

HIPCC = "/opt/rocm/bin/hipcc"


def _asm(tmp_path_factory, name: str) -> str:
    if not Path(HIPCC).exists() and shutil.which("hipcc") is None:
        pytest.skip("hipcc not available")
    import build as B

    out = tmp_path_factory.mktemp("lds") / (Path(name).stem + ".s")
    cmd = [HIPCC, *B.COMMON_FLAGS, *B.FILE_FLAGS.get(name, []), "-S", "--cuda-device-only", str(PKG / "csrc" / name),
           "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True, timeout=600)
    return out.read_text()


@pytest.mark.parametrize("name,nkernels", [("sparse_flash_mla.hip", 6), ("sparse_mla.hip", 6), ("sparse_gqa.hip", 4)])
def test_lds_waits_cover_their_reads(tmp_path_factory, name, nkernels):
    kernels, findings = asm_lds.check_asm(_asm(tmp_path_factory, name))
    assert len(kernels) >= nkernels, kernels
    assert not findings, "\n".join(map(str, findings[:20]))


def test_checker_sees_a_short_wait():
    # Sixteen reads, then a wait that leaves eight outstanding, then a use of the last one.
    body = []
    ln = 0
    for i in range(16):
        ln += 1
        body.append((ln, f"\tds_read_b128 v[{4 * i}:{4 * i + 3}], v100"))
    body += [(17, "\ts_waitcnt lgkmcnt(8)"), (18, "\tv_mfma_f32_16x16x32_f16 v[80:83], v[0:3], v[90:93], 0"),
             (19, "\tv_mfma_f32_16x16x32_f16 v[80:83], v[32:35], v[90:93], v[80:83]"), (20, "\ts_endpgm")]
    found = asm_lds.check_kernel("k", body)
    assert [f.line for f in found] == [19]
    # A scalar load issued first adds one to the count and may return last: lgkmcnt(8) still
    # proves the eighth read returned, and still not the ninth.
    body2 = [(0, "\ts_load_dword s4, s[0:1], 0x0")] + body[:17] + [
        (18, "\tv_mfma_f32_16x16x32_f16 v[80:83], v[28:31], v[90:93], 0"),
        (19, "\tv_mfma_f32_16x16x32_f16 v[80:83], v[32:35], v[90:93], v[80:83]"), (20, "\ts_endpgm")]
    assert [f.line for f in asm_lds.check_kernel("k", body2)] == [19]
    # Across a loop back edge: a read issued at the bottom and used at the top after no wait.
    loop = [(1, "\ts_mov_b32 s2, 0"), (2, ".LBB0_1:"), (3, "\tv_add_u32_e32 v1, v0, v3"),
            (4, "\tds_read_b32 v0, v2"), (5, "\ts_cbranch_scc1 .LBB0_1"), (6, "\ts_waitcnt lgkmcnt(0)"),
            (7, "\ts_endpgm")]
    assert [f.line for f in asm_lds.check_kernel("k", loop)] == [3]
