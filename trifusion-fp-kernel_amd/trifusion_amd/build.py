"""Compile the gfx950 HIP sources into the in-tree C-ABI library.

``build_library()`` drives ``hipcc`` directly (no torch extension machinery):
every ``csrc/*.hip`` file becomes an object under ``_build/`` and the objects
are linked into ``trifusion_amd/libtrifusion_amd.so``, which ``_lib.py`` loads
with ctypes. The library exports only the ``extern "C"`` entry points declared
in ``include/trifusion_amd.h``.
"""

import os
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
PROJECT_DIR = PACKAGE_DIR.parent
REPO_DIR = PROJECT_DIR.parent
CSRC_DIR = PROJECT_DIR / "csrc"
INCLUDE_DIR = REPO_DIR / "include"
BUILD_DIR = PROJECT_DIR / "_build"
LIB_PATH = PACKAGE_DIR / "libtrifusion_amd.so"
ARCH = "gfx950"

# Packed-fp32 VALU forms are disabled for all device code; hipcc -O3 would
# otherwise form them from ordinary float code.
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
COMMON_FLAGS = [f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function"]


def hipcc_path():
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    for candidate in (shutil.which("hipcc"), os.path.join(rocm, "bin", "hipcc")):
        if candidate and os.path.exists(candidate):
            return candidate
    raise RuntimeError("hipcc not found: the gfx950 kernels need ROCm's hipcc to build")


def sources():
    return sorted(CSRC_DIR.glob("*.hip"))


def _compile(hipcc, src, obj):
    cmd = [hipcc, *COMMON_FLAGS, *DEVICE_FLAGS, "-I", str(INCLUDE_DIR), "-I", str(CSRC_DIR), "-c", str(src),
           "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    lines = [
        line
        for line in (proc.stdout + proc.stderr).splitlines()
        if "is not a recognized feature for this target" not in line
    ]
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n" + "\n".join(lines))
    return lines


def build_library(verbose=False, jobs=None):
    """Compile every ``csrc/*.hip`` for gfx950 and link the shared library."""
    hipcc = hipcc_path()
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    srcs = sources()
    objs = [BUILD_DIR / (s.stem + ".o") for s in srcs]
    jobs = jobs or min(len(srcs), max(1, (os.cpu_count() or 2)))
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        logs = list(pool.map(lambda so: _compile(hipcc, *so), zip(srcs, objs)))
    if verbose:
        for src, lines in zip(srcs, logs):
            for line in lines:
                print(f"[{src.name}] {line}")
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError("link failed:\n" + proc.stdout + proc.stderr)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build_library(verbose=True))
