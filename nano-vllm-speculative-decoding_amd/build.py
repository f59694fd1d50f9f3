"""Build recipe of libnvs_amd.so: every csrc/*.hip compiled by hipcc for gfx950 and linked into one shared library
next to this file. Run as a script or call build(); it always recompiles.

Flags: -O3, C++17, position independent, packed fp32 instructions disabled (v_pk_*_f32 are not emitted), device
code for gfx950 only. The compiler's resource remarks are read back: a benchmarked kernel that spills vector
registers to private memory is reported.
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


# Kernels the benchmarked workloads run: each must keep its vector registers within budget (no spills to private
# memory), since a spill there costs more than most changes gain. Matched against the mangled kernel names.
HOT_KERNELS = (
    "attn_split_kernelILi1E",              # verify attention, bf16
    "select_kernelILi0ELi0ELb1ELb0E",      # fused accept, fp32 logits
    "select_kernelILi1ELi0ELb1ELb0E",      # fused accept, bf16 logits
    "markov_draw_kernelILi1ELb1ELb1E",     # Markov draw, bf16 logits with bias
    "qk_norm_rope_store_kernelILi1E",      # q/k norm + RoPE + KV store, bf16
)


def _vgpr_spills_by_kernel(remarks: list[str]) -> dict[str, int]:
    """Vector registers spilled to private memory by every kernel, from the compiler's resource-usage remarks."""
    out: dict[str, int] = {}
    name = None
    for line in remarks:
        if "Function Name:" in line:
            name = line.split("Function Name:", 1)[1].split()[0]
        elif name is not None and "VGPRs Spill:" in line:
            out[name] = int(line.split("VGPRs Spill:", 1)[1].split()[0])
    return out


def _compile(src: pathlib.Path, obj: pathlib.Path) -> dict[str, int]:
    """Compile one source; returns the vector-register spills of its kernels."""
    cmd = [hipcc(), *HIPCC_FLAGS, "-Rpass-analysis=kernel-resource-usage", "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # the host pass reports the disabled target feature, and the resource remarks are parsed rather than shown;
    # everything else is shown
    noise = "is not a recognized feature for this target"
    lines = proc.stderr.splitlines()
    remarks = [line for line in lines if "[-Rpass-analysis=kernel-resource-usage]" in line]
    shown = []
    after_remark = False   # the source excerpt clang prints under a remark is dropped with it
    for line in lines:
        if noise in line:
            continue
        if "[-Rpass-analysis=kernel-resource-usage]" in line:
            after_remark = True
            continue
        if _is_remark_context(line):
            if after_remark:
                continue
        else:
            after_remark = False
        shown.append(line)
    stderr = "\n".join(shown)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{stderr}")
    if stderr.strip():
        print(stderr, file=sys.stderr)
    return _vgpr_spills_by_kernel(remarks)


def _is_remark_context(line: str) -> bool:
    """The source excerpt lines clang prints after a remark ('  123 | code' and the caret line)."""
    stripped = line.strip()
    return bool(stripped) and (stripped[0].isdigit() and " | " in line or set(stripped) <= {"|", "^", " ", "~"})


def build(verbose: bool = True) -> pathlib.Path:
    """Compile csrc/*.hip and link libnvs_amd.so into the package directory; returns its path."""
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    objs = [BUILD_DIR / (src.stem + ".o") for src in sources]
    jobs = max(1, min(len(sources), int(os.environ.get("MAX_JOBS", os.cpu_count() or 1)), 8))
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        spills: dict[str, int] = {}
        for per_source in pool.map(_compile, sources, objs):
            spills.update(per_source)
    for pattern in HOT_KERNELS:
        for name, n in sorted(spills.items()):
            if pattern in name and n > 0:
                print(f"warning: hot kernel {name} spills {n} vector registers to private memory", file=sys.stderr)
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
