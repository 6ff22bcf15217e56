"""Build the gfx950 HIP library of the attention path in-tree.

``python -m nano_vllm_ascend_amd.build`` compiles every ``csrc/*.hip`` file with
hipcc for gfx950 and links them into ``nano_vllm_ascend_amd/libnvamd.so``.
The library exports the C ABI declared in ``include/nvamd.h`` and nothing that
depends on torch, so the same file serves ctypes, a C harness or any FFI.
"""
from __future__ import annotations

import os
import re
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
CSRC_DIR = PKG_DIR / "csrc"
INCLUDE_DIR = REPO_DIR / "include"
LIB_PATH = PKG_DIR / "libnvamd.so"
OBJ_DIR = PKG_DIR / "_build"

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# -packed-fp32-ops: keep the compiler from emitting packed fp32 VALU forms.
DEVICE_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    f"-I{INCLUDE_DIR}",
    f"-I{CSRC_DIR}",
]


def sources() -> list[Path]:
    return sorted(CSRC_DIR.glob("*.hip"))


_REMARK = re.compile(r"remark:\s+(Function Name|ScratchSize \[bytes/lane\]):\s+(\S+)")


def scratch_by_kernel(remarks: str) -> dict[str, int]:
    """Per-kernel scratch bytes per lane from the compiler's kernel-resource-usage remarks."""
    out: dict[str, int] = {}
    name = None
    for key, value in _REMARK.findall(remarks):
        if key == "Function Name":
            name = value
        elif name is not None:
            out[name] = int(value)
            name = None
    return out


def _compile(src: Path) -> Path:
    obj = OBJ_DIR / (src.stem + ".o")
    cmd = [HIPCC, *DEVICE_FLAGS, "-Rpass-analysis=kernel-resource-usage", "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stdout}\n{proc.stderr}")
    # Every kernel here is sized to its register budget; a register spill goes to scratch
    # memory and silently costs a large factor (one spill in the decode kernel: 1.38x), so
    # any scratch use fails the build.
    kernels = scratch_by_kernel(proc.stderr)
    if not kernels:
        raise RuntimeError(f"no kernel-resource-usage remarks for {src.name}")
    spilled = {k: v for k, v in kernels.items() if v}
    if spilled:
        raise RuntimeError(f"{src.name}: kernels use scratch (register spills): {spilled}")
    return obj


def build(verbose: bool = True) -> Path:
    """Compile all sources and link the shared library; returns its path."""
    if not Path(HIPCC).exists() and shutil.which(HIPCC) is None:
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    OBJ_DIR.mkdir(exist_ok=True)
    srcs = sources()
    if not srcs:
        raise RuntimeError(f"no HIP sources in {CSRC_DIR}")
    workers = max(1, min(len(srcs), int(os.environ.get("MAX_JOBS", "8"))))
    with ThreadPoolExecutor(max_workers=workers) as pool:
        objs = list(pool.map(_compile, srcs))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"[nvamd] built {LIB_PATH} from {len(srcs)} sources for {ARCH}")
    return LIB_PATH


if __name__ == "__main__":
    build()
    sys.exit(0)
