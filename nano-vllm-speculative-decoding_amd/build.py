"""Build recipe of libnvs_amd.so: every csrc/*.hip compiled by hipcc for gfx950 and linked into one shared library
next to this file. Run as a script or call build(); it always recompiles.

Flags: -O3, C++17, position independent, packed fp32 instructions disabled (v_pk_*_f32 are not emitted), device
code for gfx950 only.
"""
from __future__ import annotations

import concurrent.futures
import os
import pathlib
import shutil
import subprocess
import sys

PKG_DIR = pathlib.Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
INCLUDE = PKG_DIR.parent / "include"
LIB_NAME = "libnvs_amd.so"
BUILD_DIR = PKG_DIR.parent / "_build" / "nvs_amd"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
]


def hipcc() -> str:
    for candidate in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if candidate and os.path.exists(candidate):
            return candidate
    raise RuntimeError("hipcc not found: the ROCm toolchain is required to build libnvs_amd.so")


def _compile(src: pathlib.Path, obj: pathlib.Path) -> None:
    cmd = [hipcc(), *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # the host pass reports the disabled target feature; everything else is shown
    noise = "is not a recognized feature for this target"
    stderr = "\n".join(line for line in proc.stderr.splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{stderr}")
    if stderr.strip():
        print(stderr, file=sys.stderr)


def build(verbose: bool = True) -> pathlib.Path:
    """Compile csrc/*.hip and link libnvs_amd.so into the package directory; returns its path."""
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    objs = [BUILD_DIR / (src.stem + ".o") for src in sources]
    jobs = max(1, min(len(sources), int(os.environ.get("MAX_JOBS", os.cpu_count() or 1)), 8))
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        list(pool.map(_compile, sources, objs))
    out = PKG_DIR / LIB_NAME
    tmp = out.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, out)
    if verbose:
        print(f"built {out} from {len(sources)} sources", file=sys.stderr)
    return out


if __name__ == "__main__":
    build()
