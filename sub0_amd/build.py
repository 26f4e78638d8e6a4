"""Build recipe of libcda_hip.so (gfx950) -- run by ``__graft_entry__.build()``.

    python -m sub0_amd.build

Compiles every ``sub0_amd/csrc/*.hip`` with hipcc for gfx950 only into
``sub0_amd/_lib/libcda_hip.so`` (in-tree, so it travels with the source tree),
then ``sub0_amd/csrc/torch_ops.cpp`` (host C++, no device code) with g++
against torch's headers into ``sub0_amd/_lib/libcda_hip_torch.so``: the
``TORCH_LIBRARY`` registration over the C ABI, linked to ``libcda_hip.so`` by
its soname.  Packed-FP32 instructions are disabled for all device code.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OUT_DIR = PKG / "_lib"
LIB = OUT_DIR / "libcda_hip.so"
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CFLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fno-fast-math", "-ffp-contract=fast",
    "-Wall", "-Wno-unused-result",
]


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def build(verbose: bool = False) -> Path:
    obj_dir = OUT_DIR / "obj"
    obj_dir.mkdir(parents=True, exist_ok=True)

    def compile_one(src: Path) -> Path:
        obj = obj_dir / (src.stem + ".o")
        cmd = [HIPCC, *CFLAGS, "-c", str(src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"hipcc failed for {src.name}:\n{r.stdout}\n{r.stderr}")
        return obj

    with ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as ex:
        objs = list(ex.map(compile_one, sources()))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,-soname,libcda_hip.so",
           "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    build_torch_lib(verbose)
    return LIB


TORCH_LIB = OUT_DIR / "libcda_hip_torch.so"


def build_torch_lib(verbose: bool = False) -> Path:
    """libcda_hip_torch.so: torch_ops.cpp against torch's headers and libraries."""
    import torch
    tdir = Path(torch.__file__).resolve().parent
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cxx = os.environ.get("CXX", "g++")
    tmp = TORCH_LIB.with_suffix(".so.tmp")
    cmd = [cxx, "-std=c++17", "-O2", "-fPIC", "-shared", "-Wall", "-Wno-unused-parameter",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           f"-I{tdir / 'include'}", f"-I{tdir / 'include' / 'torch' / 'csrc' / 'api' / 'include'}",
           "-I/opt/rocm/include", str(CSRC / "torch_ops.cpp"), "-o", str(tmp),
           f"-L{tdir / 'lib'}", "-ltorch", "-ltorch_cpu", "-lc10", "-lc10_hip", "-ltorch_hip",
           f"-L{OUT_DIR}", "-lcda_hip", "-Wl,-rpath,$ORIGIN"]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"torch_ops.cpp failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, TORCH_LIB)
    return TORCH_LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
