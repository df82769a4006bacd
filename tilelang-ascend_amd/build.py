"""Build recipe for the gfx950 DSA library (``libdsa_mi355x.so``).

Compiles every ``csrc/*.hip`` with hipcc for gfx950 only and links one shared
library next to this file.  Run ``python tilelang-ascend_amd/build.py`` (or
``__graft_entry__.build()``).  The library is built in-tree so it travels with
the source tree; it is git-ignored.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
BUILD_DIR = PKG_DIR / "_build"
LIB_NAME = "libdsa_mi355x.so"
LIB_PATH = PKG_DIR / LIB_NAME
# torch.ops.dsa.* registrations (csrc/torch_ops.cpp): host C++ over the C ABI, linked against
# libdsa_mi355x.so and libtorch; built separately so the C-ABI library stays free of torch.
TORCH_OPS_PATH = PKG_DIR / "libdsa_torch_ops.so"
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# -packed-fp32-ops: never emit v_pk_{add,mul,fma}_f32 (see the toolchain notes in DESIGN).
COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-ffp-contract=fast",
    "-Wno-unused-result",
]


# Per-file extras: keep MFMA results in VGPRs.  indexer.hip's epilogue reads
# every result with VALU (AGPR results would each need a v_accvgpr_read), and
# sparse_flash_mla.hip's decode kernel rescales its O accumulators with VALU
# (in AGPRs they were copied out and back on every block).
FILE_FLAGS = {
    "indexer.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
    "sparse_flash_mla.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
}


def _compile(src: Path, verbose: bool) -> Path:
    obj = BUILD_DIR / (src.stem + ".o")
    cmd = [HIPCC, *COMMON_FLAGS, *FILE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stdout}\n{res.stderr}")
    return obj


def build(verbose: bool = False, jobs: int = 8) -> Path:
    """Compile all kernels and link the shared library; returns its path."""
    if not Path(HIPCC).exists() and shutil.which(HIPCC) is None:
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    BUILD_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    with cf.ThreadPoolExecutor(max_workers=max(1, min(jobs, len(sources)))) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose), sources))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    build_torch_ops(verbose)
    return LIB_PATH


def build_torch_ops(verbose: bool = False) -> Path:
    """Compile csrc/torch_ops.cpp (host only, g++) into libdsa_torch_ops.so."""
    import torch
    from torch.utils import cpp_extension

    torch_lib = Path(torch.__file__).resolve().parent / "lib"
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    tmp = TORCH_OPS_PATH.with_suffix(".so.tmp")
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-DUSE_ROCM",
           "-D__HIP_PLATFORM_AMD__", *[f"-I{d}" for d in cpp_extension.include_paths()], "-I/opt/rocm/include",
           str(CSRC / "torch_ops.cpp"), "-o", str(tmp), f"-L{PKG_DIR}", "-ldsa_mi355x", f"-L{torch_lib}",
           "-ltorch", "-ltorch_cpu", "-ltorch_hip", "-lc10", "-lc10_hip", "-Wl,-rpath,$ORIGIN",
           f"-Wl,-rpath,{torch_lib}"]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"torch_ops.cpp failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, TORCH_OPS_PATH)
    return TORCH_OPS_PATH


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
