"""Build ``libpackbalance_amd.so`` (the C-ABI library) for gfx950 with hipcc.

Every ``csrc/*.hip`` and ``csrc/*.cpp`` file is compiled to an object in
``_build/`` (in parallel), then linked into ``packbalance_amd/libpackbalance_amd.so``.
The library has no PyTorch dependency: Python reaches it through ctypes.

    python -m packbalance_amd.build            # build (always recompiles)
    python -m packbalance_amd.build --if-stale # rebuild only if a source is newer
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
INCLUDE = PKG.parent / "include"
BUILD = PKG / "_build"
LIB = PKG / "libpackbalance_amd.so"
ARCH = os.environ.get("PB_OFFLOAD_ARCH", "gfx950")

# -packed-fp32-ops: keep the compiler from emitting packed fp32 VALU ops.
COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
    f"-I{INCLUDE}",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build packbalance_amd)")


def sources() -> list[Path]:
    return sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.cpp")))


def _headers() -> list[Path]:
    return sorted(list(CSRC.glob("*.hpp")) + list(INCLUDE.glob("*.h")))


def _compile(src: Path) -> Path:
    obj = BUILD / (src.name + ".o")
    cmd = [_hipcc(), *COMMON_FLAGS, "-c", str(src), "-o", str(obj)]
    if src.suffix == ".hip":
        cmd[1:1] = ["-x", "hip"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stdout}\n{res.stderr}")
    return obj


def is_stale() -> bool:
    if not LIB.exists():
        return True
    t = LIB.stat().st_mtime
    return any(p.stat().st_mtime > t for p in sources() + _headers())


def _check_kernel_stubs(lib: Path) -> None:
    """Fail the build when a kernel's host stub is referenced but missing.

    clang's HIP host pass can silently omit the stub of a __global__ template
    (seen with a struct declared inside the kernel, or a lambda call inside a
    generic lambda's builtin argument); the library then links but fails to
    load with an undefined __device_stub__ symbol.
    """
    nm = shutil.which("nm") or "/opt/rocm/llvm/bin/llvm-nm"
    res = subprocess.run([nm, "-D", "--undefined-only", str(lib)], capture_output=True, text=True)
    missing = [ln.split()[-1] for ln in res.stdout.splitlines() if "__device_stub__" in ln]
    if missing:
        raise RuntimeError("kernel host stubs missing from the library: " + ", ".join(missing))


def build(jobs: int | None = None, verbose: bool = False) -> Path:
    BUILD.mkdir(exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), os.cpu_count() or 4, 8)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    _check_kernel_stubs(tmp)
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources", flush=True)
    return LIB


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--if-stale", action="store_true")
    ap.add_argument("-j", "--jobs", type=int, default=None)
    args = ap.parse_args()
    if args.if_stale and not is_stale():
        print(f"{LIB} is up to date")
        return
    build(args.jobs, verbose=True)


if __name__ == "__main__":
    sys.exit(main())
