"""Build libmhc_hip.so (gfx950) from ../csrc with hipcc.

Each .hip file is compiled to an object in parallel, then linked into one
shared library next to this file.  Run as ``python -m mhc_mlx_amd._build``
(with ``mhc-mlx_amd`` on sys.path) or through ``__graft_entry__.build()``.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import time
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR.parent / "csrc"
INCLUDE = PKG_DIR.parent.parent / "include"
LIB_NAME = "libmhc_hip.so"
LIB_PATH = PKG_DIR / LIB_NAME
OFFLOAD_ARCH = os.environ.get("MHC_OFFLOAD_ARCH", "gfx950")

SOURCES = ["capi.hip", "sinkhorn.hip", "fused_fwd.hip", "fused_bwd.hip", "stream_mix.hip", "generic.hip", "residual.hip",
           "mfma32.hip", "mix32.hip", "noalloc.hip"]

# Packed-FP32 VALU forms are disabled for every device pass (hipcc only; the
# host pass prints a harmless "not a recognized feature" warning).
HIP_FLAGS = [
    f"--offload-arch={OFFLOAD_ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def _compile(hipcc: str, src: Path, obj: Path) -> None:
    cmd = [hipcc, *HIP_FLAGS, f"-I{INCLUDE}", "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        msg = "\n".join(l for l in proc.stderr.splitlines() if "packed-fp32-ops" not in l)
        raise RuntimeError(f"hipcc failed for {src.name}:\n{msg}")


EXT_NAME = "_mhc_torch"
EXT_PATH = PKG_DIR / (EXT_NAME + ".so")


def build_ext(verbose: bool = True) -> Path:
    """Compile the torch binding (csrc/torch_ext.cpp) into _mhc_torch.so next to libmhc_hip.so.

    A plain C++ torch extension (g++, torch's headers and c10_hip for the current HIP stream); its
    calls into libmhc_hip resolve against the library, which _lib.load() opens with RTLD_GLOBAL
    before the binding is imported.
    """
    import torch
    import torch.utils.cpp_extension as ce

    from . import _lib

    _lib.load()
    t0 = time.time()
    bdir = PKG_DIR.parent / "_build" / "torch_ext"
    bdir.mkdir(parents=True, exist_ok=True)
    torch_lib = Path(torch.__file__).resolve().parent / "lib"
    rocm = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
    ce.load(name=EXT_NAME, sources=[str(CSRC / "torch_ext.cpp")],
            extra_include_paths=[str(INCLUDE), str(rocm / "include")],
            extra_cflags=["-O2", "-D__HIP_PLATFORM_AMD__=1"],
            extra_ldflags=[f"-L{torch_lib}", "-lc10_hip"],
            build_directory=str(bdir), verbose=False, is_python_module=True)
    built = bdir / (EXT_NAME + ".so")
    tmp = EXT_PATH.with_suffix(".so.tmp")
    shutil.copyfile(built, tmp)
    os.replace(tmp, EXT_PATH)
    if verbose:
        print(f"[mhc_mlx_amd] built {EXT_PATH} in {time.time() - t0:.1f}s", file=sys.stderr)
    return EXT_PATH


def build(verbose: bool = True, jobs: int | None = None) -> Path:
    """Compile every HIP source for gfx950 and link libmhc_hip.so. Returns its path."""
    hipcc = _hipcc()
    objdir = PKG_DIR.parent / "_build"
    objdir.mkdir(exist_ok=True)
    t0 = time.time()
    srcs = [CSRC / s for s in SOURCES]
    objs = [objdir / (s.stem + ".o") for s in srcs]
    jobs = jobs or min(len(srcs), max(1, (os.cpu_count() or 4)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        futs = [ex.submit(_compile, hipcc, s, o) for s, o in zip(srcs, objs)]
        for f in futs:
            f.result()
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={OFFLOAD_ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"[mhc_mlx_amd] built {LIB_PATH} in {time.time() - t0:.1f}s", file=sys.stderr)
    return LIB_PATH


if __name__ == "__main__":
    build()
    build_ext()
