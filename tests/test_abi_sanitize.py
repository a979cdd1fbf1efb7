"""The C ABI's host code under AddressSanitizer and UndefinedBehaviorSanitizer (CPU, no GPU).

The library is rebuilt into a temporary directory with only its host code instrumented (each sanitizer flag goes
after -Xarch_host, so the gfx950 code is the usual build), and tests/abi_sanitize_driver.c runs the size queries and
the argument checks of every entry point against it.  The driver is built with ROCm's clang, the compiler of the
library's host code, so both link the same sanitizer runtimes.  Leak detection is off: the HIP runtime keeps its
allocations until exit.
"""

import os
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
CSRC = ROOT / "moe-stream-mac_amd" / "csrc"
HIPCC = "/opt/rocm/bin/hipcc"
CLANG = "/opt/rocm/llvm/bin/clang"


@pytest.mark.skipif(not (os.path.exists(HIPCC) and os.path.exists(CLANG)), reason="ROCm compilers not present")
def test_abi_host_code_under_asan_and_ubsan(tmp_path):
    lib = tmp_path / "libgdn_san.so"
    san = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
           "-Xarch_host", "-fno-sanitize-recover=undefined", "-Xarch_host", "-fno-omit-frame-pointer"]
    cmd = [HIPCC, "--offload-arch=gfx950", "-O1", "-g", "-std=c++17", "-shared", "-fPIC",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", *san, f"-I{ROOT / 'include'}",
           *sorted(str(p) for p in CSRC.glob("*.hip")), "-o", str(lib)]
    subprocess.run(cmd, check=True, capture_output=True, timeout=900)
    exe = tmp_path / "abi_driver"
    subprocess.run([CLANG, "-g", "-O1", "-fsanitize=address,undefined", "-fno-sanitize-recover=undefined",
                    f"-I{ROOT / 'include'}", str(ROOT / "tests" / "abi_sanitize_driver.c"), str(lib),
                    f"-Wl,-rpath,{tmp_path}", "-lstdc++", "-o", str(exe)], check=True, capture_output=True,
                   timeout=300)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:halt_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1", HIP_VISIBLE_DEVICES="")
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300, env=env)
    out = res.stdout + res.stderr
    assert res.returncode == 0, out[-4000:]
    assert "abi checks passed" in res.stdout
    assert "runtime error" not in out and "AddressSanitizer" not in out, out[-4000:]
