"""Build libcqgdn.so (gfx950 HIP kernels + the C ABI of include/cqgdn.h) and its PyTorch-ROCm
operator library libcqgdn_torch.so (csrc/torch_ops.cpp, TORCH_LIBRARY(cqgdn)) in-tree.

Usage: python cq-pretrain_amd/build.py [--jobs N]

Every csrc/*.hip is compiled to an object under _build/ (git-ignored), then linked
into cqgdn/libcqgdn.so next to the Python host package, so the library travels
with the source tree.  hipcc cross-compiles for gfx950 without a GPU.  The operator
library is host C++ against the installed PyTorch-ROCm headers, compiled with the
host compiler and linked to libcqgdn.so (found next to it at run time).
"""

from __future__ import annotations

import argparse
import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
OUT = PKG / "cqgdn" / "libcqgdn.so"
OPS_OUT = PKG / "cqgdn" / "libcqgdn_torch.so"
BUILD = PKG / "_build"

ARCH = os.environ.get("CQGDN_ARCH", "gfx950")
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # never let the compiler emit packed-fp32 VALU ops (v_pk_*_f32)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # keep MFMA accumulators in VGPRs: the scans update their state with VALU
    # ops every step, which would otherwise cost an AGPR round trip per value
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found: the ROCm toolchain is required to build libcqgdn")
    return path


def _compile(src: Path, extra: list[str]) -> Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [hipcc(), *FLAGS, *extra, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(line for line in proc.stderr.splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{err}")
    if err.strip():
        print(err, file=sys.stderr)
    return obj


def build(jobs: int | None = None, extra: list[str] | None = None, verbose: bool = True) -> Path:
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    extra = list(extra or [])
    jobs = jobs or min(8, len(sources))
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        objects = list(pool.map(lambda s: _compile(s, extra), sources))
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,-soname,libcqgdn.so", "-o", str(tmp),
           *map(str, objects)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT.relative_to(ROOT)} from {len(sources)} sources for {ARCH}")
    build_ops(verbose)
    return OUT


def build_ops(verbose: bool = True) -> Path:
    """csrc/torch_ops.cpp -> cqgdn/libcqgdn_torch.so, linked to libcqgdn.so (rpath $ORIGIN)."""
    import torch
    from torch.utils import cpp_extension

    torch_dir = Path(torch.__file__).resolve().parent
    includes = [torch_dir / "include", torch_dir / "include" / "torch" / "csrc" / "api" / "include",
                Path("/opt/rocm/include"), INCLUDE]
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    tmp = OPS_OUT.with_suffix(".so.tmp")
    cmd = [os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-shared", "-fPIC", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", *(f"-I{p}" for p in includes),
           str(CSRC / "torch_ops.cpp"), "-o", str(tmp),
           *(f"-L{p}" for p in cpp_extension.library_paths()), "-lc10", "-lc10_hip", "-ltorch_cpu",
           f"-L{OUT.parent}", "-lcqgdn", "-Wl,-rpath,$ORIGIN"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"torch_ops.cpp failed to build:\n{proc.stderr}")
    os.replace(tmp, OPS_OUT)
    if verbose:
        print(f"built {OPS_OUT.relative_to(ROOT)} (TORCH_LIBRARY cqgdn)")
    return OPS_OUT


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--resource-usage", action="store_true", help="print per-kernel register/LDS usage")
    args = ap.parse_args()
    extra = ["-Rpass-analysis=kernel-resource-usage"] if args.resource_usage else []
    build(args.jobs, extra)


if __name__ == "__main__":
    main()
