"""Builds the gfx950 library and the ``langburst_cuda`` Python module in-tree.

Outputs (git-ignored, they travel with the source tree):

* ``neurova_amd/lib/liblangburst_lowbit.so`` -- the C-ABI library
  (``include/langburst_lowbit.h``), HIP kernels compiled for gfx950 only;
* ``neurova_amd/_ext/langburst_cuda.so`` -- the PyTorch-ROCm binding.

The C-ABI library records ``libamdhip64.so`` (the unversioned name PyTorch-ROCm
ships) as its HIP runtime dependency, so inside a PyTorch process it binds to
the runtime PyTorch already loaded instead of a second copy; standalone it
resolves through ``/opt/rocm/lib``.

Usage: ``python -m neurova_amd.build`` (also called by ``__graft_entry__.build``).
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB_DIR = PKG / "lib"
EXT_DIR = PKG / "_ext"
LIB = LIB_DIR / "liblangburst_lowbit.so"
EXT = EXT_DIR / "langburst_cuda.so"

ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
HIPCC = str(ROCM / "bin" / "hipcc")
ARCH = "gfx950"

HIP_SOURCES = ["lb_rowwise.hip", "lb_marlin.hip", "lb_probe.hip", "lb_noalloc.hip"]
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-result",
    # keep hipcc from emitting packed-fp32 (v_pk_*_f32) instructions
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-ffp-contract=fast",
    # gfx950 preloads the first 16 dwords of scalar kernel arguments into
    # SGPRs at wave launch: the first loads need no kernarg fetch
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
]


def _torch_paths():
    import torch.utils.cpp_extension as ce

    try:
        inc = ce.include_paths(device_type="cuda")
        libs = ce.library_paths(device_type="cuda")
    except TypeError:  # older signature
        inc = ce.include_paths(True)
        libs = ce.library_paths(True)
    return inc, libs


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in proc.stdout.splitlines() if "packed-fp32-ops" not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out)


def _torch_hip_runtime() -> Path:
    import torch

    p = Path(torch.__file__).resolve().parent / "lib" / "libamdhip64.so"
    if not p.exists():
        raise RuntimeError(f"PyTorch-ROCm HIP runtime not found at {p}")
    return p


def build_library(verbose: bool = True) -> Path:
    BUILD.mkdir(parents=True, exist_ok=True)
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    objs = []
    cmds = []
    for src in HIP_SOURCES:
        obj = BUILD / (Path(src).stem + ".o")
        objs.append(obj)
        cmds.append([HIPCC, *HIP_FLAGS, "-I", str(ROOT / "include"), "-c", str(CSRC / src), "-o", str(obj)])
    with ThreadPoolExecutor(max_workers=len(cmds)) as ex:
        list(ex.map(_run, cmds))
    hip_rt = _torch_hip_runtime()
    tmp = LIB.with_suffix(".so.tmp")
    _run([
        "g++", "-shared", "-o", str(tmp), *map(str, objs),
        f"-L{hip_rt.parent}", "-l:libamdhip64.so",
        f"-Wl,-rpath,{ROCM / 'lib'}", "-Wl,--no-undefined", "-Wl,-soname,liblangburst_lowbit.so",
    ])
    os.replace(tmp, LIB)
    if verbose:
        print(f"[neurova_amd] built {LIB}")
    return LIB


def build_extension(verbose: bool = True) -> Path:
    inc, libs = _torch_paths()
    EXT_DIR.mkdir(parents=True, exist_ok=True)
    BUILD.mkdir(parents=True, exist_ok=True)
    py_inc = sysconfig.get_paths()["include"]
    obj = BUILD / "langburst_ext.o"
    import torch

    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    _run([
        "g++", "-O2", "-std=c++17", "-fPIC", "-w",
        "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
        "-DTORCH_EXTENSION_NAME=langburst_cuda", "-DTORCH_API_INCLUDE_EXTENSION_H",
        *[f"-I{p}" for p in inc], f"-I{py_inc}", f"-I{ROOT / 'include'}",
        "-c", str(CSRC / "langburst_ext.cpp"), "-o", str(obj),
    ])
    tmp = EXT.with_suffix(".so.tmp")
    _run([
        "g++", "-shared", "-o", str(tmp), str(obj),
        f"-L{LIB_DIR}", "-llangburst_lowbit",
        *[f"-L{p}" for p in libs], "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip", "-ltorch_python",
        f"-L{_torch_hip_runtime().parent}", "-l:libamdhip64.so",
        "-Wl,-rpath,$ORIGIN/../lib", *[f"-Wl,-rpath,{p}" for p in libs],
    ])
    os.replace(tmp, EXT)
    if verbose:
        print(f"[neurova_amd] built {EXT}")
    return EXT


def build(verbose: bool = True) -> None:
    if shutil.which(HIPCC) is None and not Path(HIPCC).exists():
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    build_library(verbose)
    build_extension(verbose)


if __name__ == "__main__":
    build()
    sys.exit(0)
