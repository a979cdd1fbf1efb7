"""Builds libgdn_mi355x.so (all HIP sources under csrc/) in place for gfx950 with hipcc.

    python moe-stream-mac_amd/build.py          # or __graft_entry__.build()

Each source is compiled to an object in a temporary directory (in parallel), then the objects are linked.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
LIB = HERE / "libgdn_mi355x.so"
ARCH = os.environ.get("GDN_OFFLOAD_ARCH", "gfx950")
NOISE = "is not a recognized feature for this target"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found; the GDN engine needs ROCm's hipcc to build")


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def compile_flags() -> list[str]:
    return [f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
            # packed-FP32 VALU forms stay off (plain fp32 FMA only)
            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
            "-Wall", "-Wno-unused-result", f"-I{HERE.parent / 'include'}"]


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in res.stderr.splitlines() if NOISE not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{err}")
    if err.strip() and verbose:
        print(err, file=sys.stderr)


def build(verbose: bool = False) -> Path:
    """Compile every csrc/*.hip into one shared library; always recompiles."""
    hc, flags = hipcc(), compile_flags()
    with tempfile.TemporaryDirectory(prefix="gdn_build_") as tmpdir:
        objs = [str(Path(tmpdir) / (src.stem + ".o")) for src in sources()]
        jobs = max(1, min(len(objs), int(os.environ.get("MAX_JOBS", os.cpu_count() or 4))))
        with ThreadPoolExecutor(jobs) as ex:
            list(ex.map(lambda so: _run([hc, *flags, "-c", str(so[0]), "-o", so[1]], verbose),
                        zip(sources(), objs)))
        tmp = LIB.with_name(LIB.name + ".tmp")
        _run([hc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", str(tmp)], verbose)
        os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
