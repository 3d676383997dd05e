"""Build the package's native libraries in-tree (``python mdl_amd/build.py``;
run as a script, so that importing the package, which loads the libraries,
is not needed to build them):

* ``libmdl_hip.so``: the gfx950 HIP kernels and their C ABI (hipcc,
  ``mdl_amd/csrc/Makefile``);
* ``libmdl_torch.so``: the PyTorch-ROCm extension that defines the
  ``mdl_hip`` torch.library operators over that C ABI (g++ against the
  installed torch's headers and libraries, ``mdl_amd/csrc/torch_ops.cpp``).
"""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

CSRC = Path(__file__).resolve().parent / "csrc"
PKG = CSRC.parent
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))


def build_hip(jobs: int | None = None, force: bool = True) -> Path:
    """Compile every HIP source with hipcc and link libmdl_hip.so."""

    jobs = jobs or min(8, os.cpu_count() or 1)
    if force:
        subprocess.run(["make", "-C", str(CSRC), "clean"], check=True, stdout=subprocess.DEVNULL)
    subprocess.run(["make", "-C", str(CSRC), f"-j{jobs}"], check=True)
    out = PKG / "libmdl_hip.so"
    if not out.exists():
        raise RuntimeError("hipcc build finished without producing libmdl_hip.so")
    return out


def torch_extension_command(out: Path) -> list[str]:
    """The g++ line of libmdl_torch.so: torch's headers and ABI, HIP's
    headers (for the current-stream API), linked against torch, c10_hip and
    libmdl_hip.so (found next to it at run time)."""

    import torch
    from torch.utils.cpp_extension import include_paths, library_paths

    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1"]
    cmd += [f"-I{p}" for p in include_paths()] + [f"-I{ROCM / 'include'}"]
    cmd += [str(CSRC / "torch_ops.cpp"), "-o", str(out)]
    cmd += [f"-L{p}" for p in library_paths()] + [f"-L{PKG}"]
    cmd += ["-ltorch", "-ltorch_cpu", "-ltorch_hip", "-lc10", "-lc10_hip", "-lmdl_hip", "-Wl,-rpath,$ORIGIN"]
    cmd += [f"-Wl,-rpath,{p}" for p in library_paths()]
    return cmd


def build_torch_extension() -> Path:
    out = PKG / "libmdl_torch.so"
    tmp = out.with_suffix(".so.tmp")
    subprocess.run(torch_extension_command(tmp), check=True)
    tmp.replace(out)
    return out


def build(jobs: int | None = None, force: bool = True) -> Path:
    """Both libraries; returns libmdl_hip.so's path."""

    out = build_hip(jobs, force)
    build_torch_extension()
    return out


if __name__ == "__main__":
    print(build(force="--incremental" not in sys.argv))
