"""The C ABI's host code under AddressSanitizer and UndefinedBehaviorSanitizer (CPU only).

Builds the library's sources with -fsanitize=address,undefined on the host
compile only (the device code is built as usual; the checks launch nothing), links them with tests/sanitize/capi_host_check.cpp and runs the
driver: the chunk table on exact-size heap buffers, workspace sizes and buffer
offsets over a grid of sizes, and every entry point's rejection paths.  Any
sanitizer report or failed check fails the test.
"""

from __future__ import annotations

import os
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
CSRC = ROOT / "cq-pretrain_amd" / "csrc"
SOURCES = ["capi", "gdn_fwd", "gdn_bwd", "gdn_misc", "gdn_glue", "gdn_conv", "timer"]


def _tool(name):
    path = shutil.which(name) or f"/opt/rocm/bin/{name}"
    return path if os.path.exists(path) else None


@pytest.mark.timeout(300)
def test_capi_host_code_under_sanitizers(tmp_path):
    hipcc, clang = _tool("hipcc"), "/opt/rocm/llvm/bin/clang++"
    if hipcc is None or not os.path.exists(clang):
        pytest.skip("ROCm toolchain not found")
    inc = [f"-I{ROOT / 'include'}", f"-I{CSRC}"]
    objs, procs = [], []
    for name in SOURCES:  # the sanitizers instrument the host compile only (-Xarch_host)
        obj = tmp_path / f"{name}.o"
        cmd = [hipcc, "--offload-arch=gfx950", "-O1", "-g", "-std=c++17", "-fPIC",
               "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
               "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
               "-Xarch_host", "-fno-sanitize-recover=undefined", *inc, "-c", str(CSRC / f"{name}.hip"), "-o", str(obj)]
        procs.append(subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True))
        objs.append(str(obj))
    for proc in procs:
        _, err = proc.communicate(timeout=240)
        assert proc.returncode == 0, err
    exe = tmp_path / "capi_host_check"
    link = [clang, "-O1", "-g", "-std=c++17", "-fsanitize=address,undefined", "-fno-sanitize-recover=undefined",
            *inc, str(ROOT / "tests" / "sanitize" / "capi_host_check.cpp"), *objs,
            "-L/opt/rocm/lib", "-lamdhip64", "-Wl,-rpath,/opt/rocm/lib", "-o", str(exe)]
    subprocess.run(link, check=True, capture_output=True, text=True)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=0", UBSAN_OPTIONS="print_stacktrace=1")
    env.pop("LD_PRELOAD", None)
    run = subprocess.run([str(exe)], capture_output=True, text=True, env=env, timeout=120)
    assert run.returncode == 0, run.stdout + run.stderr
    assert "capi host checks passed" in run.stdout
    assert "runtime error" not in run.stderr and "AddressSanitizer" not in run.stderr, run.stderr
