"""Build libquail_mi355x.so, the C-ABI library of gfx950 kernels, in-tree.

`python -m quail_amd.build` compiles every `csrc/*.hip` with hipcc for
gfx950 and every host-only `csrc/*.cpp` (the packing runtime) with g++, and
links them into `quail_amd/libquail_mi355x.so`. The library has no torch
dependency; Python reaches it through ctypes (quail_amd/_lib.py).
"""

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
LIB = HERE / "libquail_mi355x.so"
BUILD = HERE / "_build"
ARCH = "gfx950"

FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
    # no packed fp32 VALU ops (v_pk_*_f32) anywhere in the device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    for candidate in (os.environ.get("HIPCC"), shutil.which("hipcc"),
                      "/opt/rocm/bin/hipcc"):
        if candidate and Path(candidate).exists():
            return candidate
    raise RuntimeError("hipcc not found; the gfx950 kernels cannot be built")


HOST_FLAGS = ["-O3", "-fPIC", "-std=c++17", "-Wall"]


def _compile(src: Path, obj: Path) -> None:
    if src.suffix == ".cpp":
        # host-only C++ (the packing runtime): the system compiler
        cmd = [shutil.which("g++") or "g++", *HOST_FLAGS, "-I", str(CSRC), "-c", str(src),
               "-o", str(obj)]
    else:
        cmd = [hipcc(), *FLAGS, "-I", str(CSRC), "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"{cmd[0]} failed on {src.name}:\n{proc.stderr}")


def build(verbose: bool = False) -> Path:
    """Compile and link the library; returns its path."""
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    objects = [BUILD / (src.name.replace(".", "_") + ".o") for src in sources]
    workers = min(len(sources), max(1, min(8, os.cpu_count() or 1)))
    with concurrent.futures.ThreadPoolExecutor(workers) as pool:
        futures = [pool.submit(_compile, s, o) for s, o in zip(sources, objects)]
        for future in futures:
            future.result()
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
           *map(str, objects)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(sources)} sources", file=sys.stderr)
    return LIB


if __name__ == "__main__":
    build(verbose=True)
