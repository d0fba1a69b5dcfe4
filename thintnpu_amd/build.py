"""Build recipe for the gfx950 HIP library and the PyTorch PrivateUse1 glue.

Everything is built in-tree:
  thintnpu_amd/libthin_hip.so        C-ABI kernel library (include/thin_hip.h), hipcc
  thintnpu_amd/capi_selftest         plain C consumer of the C ABI (no PyTorch), gcc
  thin_backend/lib*.so               PrivateUse1 registrations (libtorch + HIP runtime), g++

Run ``python -m thintnpu_amd.build`` (or ``__graft_entry__.build()``).  Every
call recompiles; objects go to ``_build/`` at the repository root.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import sysconfig
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
PKG = ROOT / "thintnpu_amd"
HIP_SRC = PKG / "csrc" / "hip"
TORCH_SRC = PKG / "csrc" / "torch"
INCLUDE = ROOT / "include"
BUILD = ROOT / "_build"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
HIPCC = str(ROCM / "bin" / "hipcc")
ARCH = os.environ.get("THIN_OFFLOAD_ARCH", "gfx950")

HIP_LIB = PKG / "libthin_hip.so"

# Device flags: gfx950 only, code object v5 (loadable by the HIP runtime that
# ships with PyTorch), packed-fp32 instruction selection disabled.
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-mcode-object-version=5",
    # No implicit contraction: only explicit fmaf() fuses, so every fp16 rounding
    # the kernels spell out (e.g. the unfused-chain intermediates) survives.
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-result",
    f"-I{INCLUDE}", f"-I{HIP_SRC}",
]


def _run(cmd: list[str], cwd: Path | None = None) -> None:
    proc = subprocess.run(cmd, cwd=cwd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in proc.stdout.splitlines()
                    if "packed-fp32-ops" not in l and "not a recognized feature" not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out, file=sys.stderr)


def _jobs() -> int:
    return max(1, min(8, int(os.environ.get("MAX_JOBS", os.cpu_count() or 4))))


def build_hip(verbose: bool = False) -> Path:
    """Compile every csrc/hip source with hipcc and link libthin_hip.so."""
    obj_dir = BUILD / "hip"
    obj_dir.mkdir(parents=True, exist_ok=True)
    sources = sorted(list(HIP_SRC.glob("*.hip")) + list(HIP_SRC.glob("*.cpp")))

    def compile_one(src: Path) -> Path:
        obj = obj_dir / (src.name + ".o")
        cmd = [HIPCC, *HIP_FLAGS, "-x", "hip", "-c", str(src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), file=sys.stderr)
        _run(cmd)
        return obj

    with cf.ThreadPoolExecutor(_jobs()) as pool:
        objs = list(pool.map(compile_one, sources))
    tmp = HIP_LIB.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp),
          f"-Wl,-rpath,{ROCM / 'lib'}"])
    os.replace(tmp, HIP_LIB)
    return HIP_LIB


SELFTEST = PKG / "capi_selftest"


def build_selftest(verbose: bool = False) -> Path:
    """A plain C program over include/thin_hip.h (no PyTorch): hipMalloc'd
    buffers, its own stream, exact checks on the host."""
    cc = os.environ.get("CC", "gcc")
    cmd = [cc, "-std=c11", "-O2", "-Wall", "-D__HIP_PLATFORM_AMD__", f"-I{ROCM / 'include'}", f"-I{INCLUDE}",
           str(PKG / "csrc" / "capi_selftest.c"), "-o", str(SELFTEST) + ".tmp", f"-L{HIP_LIB.parent}", "-lthin_hip",
           f"-L{ROCM / 'lib'}", "-lamdhip64", "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{ROCM / 'lib'}"]
    if verbose:
        print(" ".join(cmd), file=sys.stderr)
    _run(cmd)
    os.replace(str(SELFTEST) + ".tmp", SELFTEST)
    return SELFTEST


def build(verbose: bool = False) -> None:
    build_hip(verbose)
    build_selftest(verbose)
    try:
        from thintnpu_amd import torch_build  # noqa: F401  (glue recipe, optional until present)
    except ImportError:
        return
    torch_build.build(verbose)


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
    print("built", HIP_LIB)
