"""Build the reference's own ATen implementation of the path into oracle/_ref/
(test infrastructure only).

The reference's CPU ATen backend (csrc/mxmac/attention_forward.cpp,
paged_kv.cpp, workspace.cpp: flash_attn_with_kvcache with the paged gather and
append, flash_attn_func, flash_attn_varlen_func) needs only torch's C++
headers and libraries, which this image has. This script compiles those three
files where they lie under the reference checkout with g++ (one line per
file, then the link; the reference's own CMake build is not run) into
oracle/_ref/mxfa_ref_aten<EXT_SUFFIX>, a Python module named mxfa_ref_aten.
Nothing of the reference is copied into the repository: only the built
module, which .gitignore keeps out of history, travels with the tree.

    python oracle/build_ref.py [--reference /root/reference]

Without the reference checkout (a GPU box) it does nothing and says so.
"""

from __future__ import annotations

import argparse
import concurrent.futures
import os
import subprocess
import sys
import sysconfig
from pathlib import Path

ORACLE_DIR = Path(__file__).resolve().parent
REF_DIR = ORACLE_DIR / "_ref"
MODULE = "mxfa_ref_aten"
SOURCES = ("attention_forward.cpp", "paged_kv.cpp", "workspace.cpp")


def output_path() -> Path:
    return REF_DIR / (MODULE + sysconfig.get_config_var("EXT_SUFFIX"))


def _flags() -> tuple[list[str], list[str]]:
    """(compile flags, link flags) against the installed torch."""
    import torch
    from torch.utils import cpp_extension

    torch_lib = Path(torch.__file__).resolve().parent / "lib"
    abi = int(torch.compiled_with_cxx11_abi())
    cflags = ["-O2", "-std=c++17", "-fPIC", "-fvisibility=hidden",
              f"-D_GLIBCXX_USE_CXX11_ABI={abi}", f"-DTORCH_EXTENSION_NAME={MODULE}",
              "-DTORCH_API_INCLUDE_EXTENSION_H",
              *[f"-I{p}" for p in cpp_extension.include_paths()],
              f"-I{sysconfig.get_paths()['include']}"]
    lflags = [f"-L{torch_lib}", "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python",
              f"-Wl,-rpath,{torch_lib}"]
    return cflags, lflags


def _run(cmd: list[str]) -> None:
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"oracle/_ref build failed: {' '.join(cmd)}\n{result.stdout}\n"
                           f"{result.stderr}")


def build(reference: Path = Path("/root/reference")) -> Path | None:
    """Compile the module when the reference checkout is present (one g++ per
    source in parallel, then the link); return its path."""
    src_dir = reference / "csrc" / "mxmac"
    if not (src_dir / SOURCES[0]).exists():
        print(f"oracle/_ref: no reference checkout at {reference}; nothing built", file=sys.stderr)
        return None
    REF_DIR.mkdir(exist_ok=True)
    cflags, lflags = _flags()
    objs = [REF_DIR / (Path(name).stem + ".o") for name in SOURCES]
    with concurrent.futures.ThreadPoolExecutor(max_workers=len(SOURCES)) as pool:
        jobs = [pool.submit(_run, ["g++", *cflags, f"-I{src_dir}", "-c", str(src_dir / name),
                                   "-o", str(obj)]) for name, obj in zip(SOURCES, objs)]
        for job in jobs:
            job.result()
    out = output_path()
    tmp = out.with_suffix(".tmp")
    _run(["g++", "-shared", *map(str, objs), *lflags, "-o", str(tmp)])
    os.replace(tmp, out)
    for obj in objs:
        obj.unlink()
    return out


if __name__ == "__main__":
    ap = argparse.ArgumentParser(description=__doc__,
                                 formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--reference", type=Path, default=Path("/root/reference"))
    print(build(ap.parse_args().reference))
