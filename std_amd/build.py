"""Build libstdhip.so (gfx950) in-tree with hipcc.

Usage: ``python -m std_amd.build`` or ``std_amd.build.build_library()``.
Each ``std_amd/csrc/*.hip`` file is compiled to an object in parallel, then
linked into ``std_amd/_lib/libstdhip.so``. No torch headers are involved: the
library is plain HIP C++ behind the C ABI declared in ``include/std_hip.h``.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
CSRC_DIR = PKG_DIR / "csrc"
INCLUDE_DIR = REPO_DIR / "include"
LIB_DIR = PKG_DIR / "_lib"
LIB_PATH = LIB_DIR / "libstdhip.so"
# The timing build of the same sources (phase stamps compiled in; see
# attention.hip): loaded only by ``bench.py --workload phases``.
STAMPS_LIB_PATH = LIB_DIR / "libstdhip_stamps.so"
OFFLOAD_ARCH = "gfx950"

# Packed-fp32 VALU forms are kept out of the generated code; hipcc's host
# pass warns that it does not know this feature, which is harmless.
DEVICE_FLAGS = [
    f"--offload-arch={OFFLOAD_ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found; the HIP library cannot be built")
    return path


def _compile(src: Path, obj: Path, verbose: bool, defines=()) -> None:
    cmd = [_hipcc(), *DEVICE_FLAGS, *[f"-D{d}" for d in defines], f"-I{INCLUDE_DIR}", f"-I{CSRC_DIR}", "-c", str(src),
           "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "packed-fp32-ops' is not a recognized feature"
    msgs = "\n".join(line for line in (res.stdout + res.stderr).splitlines() if noise not in line)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{msgs}")
    if verbose and msgs.strip():
        print(msgs, file=sys.stderr)


def build_library(verbose: bool = False, stamps: bool = False) -> Path:
    """Compile every HIP source and link libstdhip.so (with stamps: the timing
    build libstdhip_stamps.so); returns its path."""
    sources = sorted(CSRC_DIR.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC_DIR}")
    obj_dir = LIB_DIR / ("_build_stamps" if stamps else "_build")
    obj_dir.mkdir(parents=True, exist_ok=True)
    objs = [obj_dir / (s.stem + ".o") for s in sources]
    defines = ("STD_PHASE_STAMPS=1",) if stamps else ()
    with cf.ThreadPoolExecutor(max_workers=min(len(sources), 8)) as ex:
        list(ex.map(lambda so: _compile(so[0], so[1], verbose, defines), zip(sources, objs)))
    out = STAMPS_LIB_PATH if stamps else LIB_PATH
    tmp = out.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={OFFLOAD_ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}{res.stderr}")
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build_library(verbose="-v" in sys.argv, stamps="--stamps" in sys.argv))
