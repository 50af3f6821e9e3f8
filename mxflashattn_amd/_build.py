"""Build the gfx950 C-ABI library ``mxflashattn_amd/_lib/libmxfa_mi355x.so``.

The library is compiled in-tree with ``hipcc`` directly (no torch headers), so
it loads through ctypes from any host process. Run ``python -m
mxflashattn_amd._build`` or ``__graft_entry__.build()``.
"""

from __future__ import annotations

import concurrent.futures
import os
import re
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
SOURCES = ("split_decode.hip", "split_hd64.hip", "split_hd64_ws.hip", "split_hd64_ws4.hip",
           "split_hd128.hip", "split_hd128_ws.hip", "split_hd128_ws4.hip", "split_hd256.hip",
           "split_hd256_ws.hip", "split_hd256_ws4.hip", "kv_append.hip", "stream_read.hip")
# Comparison build: QK always on the matrix cores (the default build puts it on
# the VALU for launches of few columns at head dims >= 128).
QK_MFMA_LIB_PATH = PACKAGE_DIR / "_lib" / "qk_mfma" / "libmxfa_mi355x.so"
ARCH = "gfx950"

# Packed-fp32 VALU forms are disabled for every device pass: hipcc forms them
# from plain float code, and some of their forms have given wrong results on
# MI355X boxes with no error raised. Kernel arguments ahead of the parameter
# struct (what each kernel's first loads need) are preloaded into SGPRs at
# wave launch, so those loads do not wait for a kernarg-segment read. MFMA
# results and accumulators live in VGPRs where the kernel fits 256 of them:
# with accumulation registers the compiler put the QK scores and the PV
# accumulators in the same ones and copied the accumulators out and back on
# every tile (40 copies per tile at 16-bit HD 64).
HIPCC_FLAGS = (
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-mcode-object-version=5",
    "-mllvm",
    "-amdgpu-kernarg-preload-count=16",
    "-mllvm",
    "-amdgpu-mfma-vgpr-form",
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


def compile_command(source: Path, obj: Path, extra: tuple[str, ...] = ()) -> list[str]:
    return [hipcc_path(), *HIPCC_FLAGS, *extra, RESOURCE_REMARKS, f"-I{INCLUDE_DIR}",
            f"-I{CSRC_DIR}", "-c", str(source), "-o", str(obj)]


def link_command(objs: list[Path], output: Path) -> list[str]:
    return [hipcc_path(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o",
            str(output)]


def _run(cmd: list[str]) -> str:
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(
            f"hipcc failed ({result.returncode}): {' '.join(cmd)}\n{result.stdout}\n{result.stderr}"
        )
    return result.stderr


# Every kernel must keep its state in registers: a kernel that spills VGPRs or
# uses private (scratch) memory for any other reason fails the build. The
# compiler's resource-usage remarks (one block per kernel) are the record.
RESOURCE_REMARKS = "-Rpass-analysis=kernel-resource-usage"
_REMARK = re.compile(r"remark:\s+(Function Name|VGPRs Spill|ScratchSize \[bytes/lane\]|VGPRs|"
                     r"AGPRs|Occupancy \[waves/SIMD\]|LDS Size \[bytes/block\]): (\S+)")

# Static LDS each kernel family declares (the combine's reduction buffer; the
# split kernels' per-wave tile totals), in bytes. More than that is a private
# array the compiler moved into LDS, the same failure as scratch (a register
# array indexed at run time) in another memory: it fails the build too.
# Dynamic LDS (the tile prefix sums, the per-sequence kernel's pieces) is not
# counted in the remark.
STATIC_LDS_LIMITS = {"split_combine_kernel": 256 * 6 * 4}
STATIC_LDS_DEFAULT = 64


def resource_usage(remarks: str) -> dict[str, dict[str, str]]:
    """Kernel name -> {field: value} from kernel-resource-usage remarks."""
    kernels: dict[str, dict[str, str]] = {}
    current: dict[str, str] | None = None
    for m in _REMARK.finditer(remarks):
        field, value = m.group(1), m.group(2)
        if field == "Function Name":
            current = kernels.setdefault(value, {})
        elif current is not None:
            current[field] = value
    return kernels


def static_lds_limit(name: str) -> int:
    for family, limit in STATIC_LDS_LIMITS.items():
        if family in name:
            return limit
    return STATIC_LDS_DEFAULT


def check_resource_usage(source: str, remarks: str) -> dict[str, dict[str, str]]:
    """Raise when a kernel of ``source`` spills VGPRs, uses scratch memory or
    holds more static LDS than its family declares."""
    kernels = resource_usage(remarks)
    bad = [f"{name}: VGPR spills {u.get('VGPRs Spill')}, scratch "
           f"{u.get('ScratchSize [bytes/lane]')} bytes/lane, static LDS "
           f"{u.get('LDS Size [bytes/block]')} bytes (limit {static_lds_limit(name)})"
           for name, u in kernels.items()
           if u.get("VGPRs Spill", "0") != "0" or u.get("ScratchSize [bytes/lane]", "0") != "0"
           or int(u.get("LDS Size [bytes/block]", "0")) > static_lds_limit(name)]
    if bad:
        raise RuntimeError(f"{source}: kernels spill, use scratch memory or promote arrays to "
                           "LDS:\n" + "\n".join(bad))
    return kernels


TORCH_OP_SOURCE = CSRC_DIR / "torch_op.cpp"


def torch_op_path() -> Path:
    import sysconfig

    return LIB_DIR / ("_mxfa_torch" + sysconfig.get_config_var("EXT_SUFFIX"))


def torch_op_command(output: Path) -> list[str]:
    """g++ line of the torch operator (host code only, no device code): it
    includes torch's and HIP's headers and links torch and the C-ABI library,
    found next to it at run time ($ORIGIN)."""
    import sysconfig

    import torch
    from torch.utils import cpp_extension

    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    torch_lib = Path(torch.__file__).resolve().parent / "lib"
    abi = int(torch.compiled_with_cxx11_abi())
    return ["g++", "-O2", "-std=c++17", "-shared", "-fPIC", "-fvisibility=hidden",
            f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-D__HIP_PLATFORM_AMD__=1",
            "-DTORCH_EXTENSION_NAME=_mxfa_torch", "-DTORCH_API_INCLUDE_EXTENSION_H",
            *[f"-I{p}" for p in cpp_extension.include_paths()],
            f"-I{sysconfig.get_paths()['include']}", f"-I{rocm}/include", f"-I{INCLUDE_DIR}",
            str(TORCH_OP_SOURCE), f"-L{torch_lib}", f"-L{LIB_DIR}", "-lmxfa_mi355x", "-lc10",
            "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip", "-ltorch_python",
            f"-Wl,-rpath,{torch_lib}", "-Wl,-rpath,$ORIGIN", "-o", str(output)]


def build(verbose: bool = False, jobs: int | None = None, lib_path: Path = LIB_PATH,
          extra: tuple[str, ...] = (), torch_op: bool = True,
          check_registers: bool = True) -> Path:
    """Compile the library and the torch operator in front of it; always
    recompiles (one hipcc per source, in parallel, then one link, then the
    operator). ``lib_path`` and ``extra`` hipcc flags give other builds of the
    same sources (the profiling build of wave_timeline, whose clock stamps add
    live values and which alone passes ``check_registers=False``). Returns the
    library path."""
    lib_dir = lib_path.parent
    lib_dir.mkdir(parents=True, exist_ok=True)
    obj_dir = lib_dir / "obj"
    obj_dir.mkdir(exist_ok=True)
    objs = [obj_dir / (Path(name).stem + ".o") for name in SOURCES]
    cmds = [compile_command(CSRC_DIR / name, obj, extra) for name, obj in zip(SOURCES, objs)]
    if verbose:
        for cmd in cmds:
            print(" ".join(cmd), flush=True)
    workers = jobs or min(len(cmds), os.cpu_count() or 1)
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
        futures = [pool.submit(_run, cmd) for cmd in cmds]
        remarks = [(name, future.result()) for name, future in zip(SOURCES, futures)]
    kernels = sum(len(check_resource_usage(name, text) if check_registers
                      else resource_usage(text)) for name, text in remarks)
    if kernels == 0:
        raise RuntimeError("no kernel-resource-usage remarks from hipcc: the check saw no kernel")
    tmp = lib_path.with_suffix(".so.tmp")
    _run(link_command(objs, tmp))
    os.replace(tmp, lib_path)
    if not torch_op:
        return lib_path
    op = torch_op_path()
    op_tmp = op.with_suffix(".tmp")
    cmd = torch_op_command(op_tmp)
    if verbose:
        print(" ".join(cmd), flush=True)
    _run(cmd)
    os.replace(op_tmp, op)
    return lib_path


if __name__ == "__main__":
    if "--qk-mfma" in sys.argv:
        path = build(verbose="-v" in sys.argv, lib_path=QK_MFMA_LIB_PATH,
                     extra=("-DMXFA_QK_ON_MFMA",), torch_op=False)
    else:
        path = build(verbose="-v" in sys.argv)
    print(path)
