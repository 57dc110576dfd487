"""Build recipe for the gfx950 HIP library behind the C ABI.

Compiles every ``laprune_amd/csrc/*.hip`` with hipcc for gfx950 into
``laprune_amd/_lib/liblaprune_hip.so`` (in-tree, so the built library travels
with the source tree), then ``csrc/torch_ops.cpp`` (host code: torch custom
ops over the C ABI) with hipcc against the installed torch headers into
``laprune_amd/_lib/liblaprune_torch.so``.  No torch extension machinery
(cpp_extension, hipify) is involved.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIBDIR = PKG / "_lib"
LIBNAME = "liblaprune_hip.so"
OBJDIR = PKG / "_build"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # explicit arithmetic order: no silent a*b+c contraction anywhere
    "-ffp-contract=off",
    # no packed fp32 VALU ops (v_pk_*_f32) are emitted
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found: the gfx950 library cannot be built")
    return path


def lib_path() -> Path:
    return LIBDIR / LIBNAME


TORCH_LIBNAME = "liblaprune_torch.so"


def torch_lib_path() -> Path:
    return LIBDIR / TORCH_LIBNAME


def build_torch_ops() -> Path:
    """Compile the torch op binding (host C++) against the installed torch
    and link it to liblaprune_hip.so (found next to it at load time)."""
    import torch
    tp = Path(torch.__file__).resolve().parent
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    tmp = LIBDIR / (TORCH_LIBNAME + ".tmp")
    cmd = [hipcc(), "-x", "c++", "-O2", "-std=c++17", "-fPIC", "-shared",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           "-I/opt/rocm/include", f"-I{tp / 'include'}",
           f"-I{tp / 'include' / 'torch' / 'csrc' / 'api' / 'include'}",
           str(CSRC / "torch_ops.cpp"), "-o", str(tmp),
           f"-L{tp / 'lib'}", "-ltorch", "-ltorch_cpu", "-lc10", "-lc10_hip", "-ltorch_hip",
           f"-L{LIBDIR}", "-llaprune_hip", "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{tp / 'lib'}"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"torch op binding failed to build:\n{res.stderr}")
    os.replace(tmp, torch_lib_path())
    return torch_lib_path()


def _compile(src: Path, obj: Path) -> None:
    cmd = [hipcc(), *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stderr}")
    # the host pass does not know the packed-fp32 feature; drop that noise
    err = "\n".join(l for l in res.stderr.splitlines()
                    if "packed-fp32-ops" not in l and l.strip())
    if err:
        sys.stderr.write(err + "\n")


def build(jobs: int | None = None, verbose: bool = False) -> Path:
    """Compile all HIP sources and link the shared library; returns its path."""
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    OBJDIR.mkdir(exist_ok=True)
    LIBDIR.mkdir(exist_ok=True)
    objs = [OBJDIR / (s.stem + ".o") for s in sources]
    jobs = jobs or min(len(sources), max(1, (os.cpu_count() or 2)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        futs = [ex.submit(_compile, s, o) for s, o in zip(sources, objs)]
        for f in futs:
            f.result()
    tmp = LIBDIR / (LIBNAME + ".tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
           *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, lib_path())
    build_torch_ops()
    if verbose:
        print(f"built {lib_path()} and {torch_lib_path()}")
    return lib_path()


if __name__ == "__main__":
    build(verbose=True)
