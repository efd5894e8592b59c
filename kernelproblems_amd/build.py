"""Builds the gfx950 C-ABI library ``kernelproblems_amd/libkp_hip.so`` in-tree.

Every ``csrc/*.hip`` file is compiled with hipcc for gfx950 only (one code
object, no CUDA/host dual paths) and linked into one shared library that
exports the ``extern "C"`` entry points declared in ``include/kp.h``.
``csrc/kp_torch.cpp`` (host code, g++ against torch's headers) becomes the
Python module ``_kp_torch.so`` beside it: the native tensor-level wrappers of
the most-called entry points, linked to ``libkp_hip.so``.

Usage: ``python -m kernelproblems_amd.build`` (also called by
``__graft_entry__.build()``).  The build always recompiles.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
OBJ_DIR = PKG / "_build"
LIB_PATH = PKG / "libkp_hip.so"
EXT_PATH = PKG / "_kp_torch.so"

ARCH = "gfx950"
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # Packed fp32 ops (v_pk_{add,mul,fma}_f32) are kept out of all generated code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{ROOT / 'include'}",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the gfx950 library cannot be built")


def _compile(src: Path) -> Path:
    obj = OBJ_DIR / (src.stem + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stderr}")
    return obj


def _ext_flags():
    """g++ flags of the torch-facing wrapper module (host code only): torch's
    headers and ABI, the HIP runtime headers for the current-stream lookup."""
    import sysconfig

    import torch
    from torch.utils import cpp_extension as ce

    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    flags = ["-O2", "-std=c++17", "-fPIC", "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
             "-DTORCH_API_INCLUDE_EXTENSION_H", "-DTORCH_EXTENSION_NAME=_kp_torch", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
             "-I/opt/rocm/include", f"-I{ROOT / 'include'}", f"-I{sysconfig.get_paths()['include']}"]
    flags += [f"-I{p}" for p in ce.include_paths()]
    libs = [f"-L{p}" for p in ce.library_paths()] + ["-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_python"]
    return flags, libs


def _compile_ext() -> Path:
    flags, _ = _ext_flags()
    obj = OBJ_DIR / "kp_torch.o"
    res = subprocess.run(["g++", *flags, "-c", str(CSRC / "kp_torch.cpp"), "-o", str(obj)], capture_output=True,
                         text=True)
    if res.returncode != 0:
        raise RuntimeError(f"g++ failed for kp_torch.cpp:\n{res.stderr}")
    return obj


def build(verbose: bool = True) -> Path:
    """Compiles all HIP sources and links libkp_hip.so, then the torch-facing
    wrapper module _kp_torch.so (linked to it); returns libkp_hip.so's path."""
    OBJ_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    jobs = min(len(sources) + 1, int(os.environ.get("MAX_JOBS", "8")))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        ext_obj = ex.submit(_compile_ext)  # the slowest single file: started first
        objs = list(ex.map(_compile, sources))
        ext_obj = ext_obj.result()
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link of {LIB_PATH.name} failed:\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    _, libs = _ext_flags()
    tmp = EXT_PATH.with_suffix(".so.tmp")
    cmd = ["g++", "-shared", "-fPIC", "-o", str(tmp), str(ext_obj), f"-L{PKG}", "-lkp_hip", "-Wl,-rpath,$ORIGIN", *libs]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link of {EXT_PATH.name} failed:\n{res.stderr}")
    os.replace(tmp, EXT_PATH)
    if verbose:
        print(f"[kernelproblems_amd] built {LIB_PATH} from {len(sources)} HIP sources and {EXT_PATH.name}", flush=True)
    return LIB_PATH


if __name__ == "__main__":
    build()
    sys.exit(0)
