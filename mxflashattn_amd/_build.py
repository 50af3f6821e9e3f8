"""Build the gfx950 C-ABI library ``mxflashattn_amd/_lib/libmxfa_mi355x.so``.

The library is compiled in-tree with ``hipcc`` directly (no torch headers), so
it loads through ctypes from any host process. Run ``python -m
mxflashattn_amd._build`` or ``__graft_entry__.build()``.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
REPO_DIR = PACKAGE_DIR.parent
CSRC_DIR = PACKAGE_DIR / "csrc"
INCLUDE_DIR = REPO_DIR / "include"
LIB_DIR = PACKAGE_DIR / "_lib"
LIB_NAME = "libmxfa_mi355x.so"
LIB_PATH = LIB_DIR / LIB_NAME
SOURCES = ("split_decode.hip", "kv_append.hip")
ARCH = "gfx950"

# Packed-fp32 VALU forms are disabled for every device pass.
HIPCC_FLAGS = (
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-mcode-object-version=5",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
)


def hipcc_path() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    candidate = Path(rocm) / "bin" / "hipcc"
    if candidate.exists():
        return str(candidate)
    found = shutil.which("hipcc")
    if found is None:
        raise RuntimeError("hipcc not found: set ROCM_PATH or put hipcc on PATH")
    return found


def build_command(output: Path = LIB_PATH, extra: tuple[str, ...] = ()) -> list[str]:
    return [
        hipcc_path(),
        *HIPCC_FLAGS,
        *extra,
        f"-I{INCLUDE_DIR}",
        f"-I{CSRC_DIR}",
        *(str(CSRC_DIR / name) for name in SOURCES),
        "-o",
        str(output),
    ]


def build(verbose: bool = False) -> Path:
    """Compile the library; always recompiles. Returns the library path."""
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = build_command(tmp)
    if verbose:
        print(" ".join(cmd), flush=True)
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(
            f"hipcc failed ({result.returncode}):\n{result.stdout}\n{result.stderr}"
        )
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
