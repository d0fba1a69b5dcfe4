"""Build recipe for the PyTorch PrivateUse1 glue libraries (host C++ over the
thin_hip C ABI).  Output file names are the ones the reference's callers load
(thin_backend/libthin_backend.so, libflow_ops.so, libconv_flow.so,
libselection_flow.so, libthin_blocked.so, libbmm_flow.so, libdepthwise_flow.so).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import sys
from pathlib import Path

from thintnpu_amd.build import BUILD, HIP_LIB, INCLUDE, ROCM, ROOT, TORCH_SRC, _jobs, _run

OUT = ROOT / "thin_backend"

# library -> sources (relative to csrc/torch); libthin_backend.so first
LIBS = {
    "libthin_backend.so": ["runtime.cpp", "ops.cpp"],
    "libflow_ops.so": ["flow_ops.cpp"],
    "libconv_flow.so": ["conv_flow.cpp"],
    "libselection_flow.so": ["selection.cpp"],
    "libthin_blocked.so": ["blocked.cpp"],
    "libbmm_flow.so": ["bmm_flow.cpp"],
    "libdepthwise_flow.so": ["depthwise_flow_stub.cpp"],
}


def _torch_paths():
    import torch
    base = Path(torch.__file__).resolve().parent
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    return base, abi


def build(verbose: bool = False) -> None:
    base, abi = _torch_paths()
    obj_dir = BUILD / "torch"
    obj_dir.mkdir(parents=True, exist_ok=True)
    OUT.mkdir(exist_ok=True)
    cxx = os.environ.get("CXX", "g++")
    flags = ["-std=c++17", "-O2", "-fPIC", f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-D__HIP_PLATFORM_AMD__",
             f"-I{base / 'include'}", f"-I{base / 'include' / 'torch' / 'csrc' / 'api' / 'include'}",
             f"-I{ROCM / 'include'}", f"-I{INCLUDE}", f"-I{TORCH_SRC}", "-Wno-deprecated-declarations"]

    sources = sorted({s for srcs in LIBS.values() for s in srcs})

    def compile_one(name: str) -> None:
        cmd = [cxx, *flags, "-c", str(TORCH_SRC / name), "-o", str(obj_dir / (name + ".o"))]
        if verbose:
            print(" ".join(cmd), file=sys.stderr)
        _run(cmd)

    with cf.ThreadPoolExecutor(_jobs()) as pool:
        list(pool.map(compile_one, sources))

    torch_libs = [f"-L{base / 'lib'}", "-lc10", "-ltorch_cpu", "-ltorch"]
    hip_libs = [f"-L{ROCM / 'lib'}", "-lamdhip64"]
    rpaths = ["-Wl,-rpath,$ORIGIN", "-Wl,-rpath,$ORIGIN/../thintnpu_amd", f"-Wl,-rpath,{base / 'lib'}",
              f"-Wl,-rpath,{ROCM / 'lib'}"]
    guard = cf.ThreadPoolExecutor(1).submit(build_region_guard, verbose)
    for lib, srcs in LIBS.items():
        objs = [str(obj_dir / (s + ".o")) for s in srcs]
        extra = [] if lib == "libthin_backend.so" else [f"-L{OUT}", "-lthin_backend"]
        tmp = OUT / (lib + ".tmp")
        _run([cxx, "-shared", "-fPIC", *objs, "-o", str(tmp), *extra, f"-L{HIP_LIB.parent}", "-lthin_hip",
              *torch_libs, *hip_libs, *rpaths])
        os.replace(tmp, OUT / lib)
    guard.result()


def build_region_guard(verbose: bool = False) -> Path:
    """pybind11 extension thin_backend/_region_guard<EXT_SUFFIX> (host C++ only)."""
    import sysconfig
    base, abi = _torch_paths()
    suffix = sysconfig.get_config_var("EXT_SUFFIX")
    target = OUT / ("_region_guard" + suffix)
    cxx = os.environ.get("CXX", "g++")
    cmd = [cxx, "-std=c++17", "-O2", "-shared", "-fPIC", "-fvisibility=hidden", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           f"-I{sysconfig.get_paths()['include']}", f"-I{base / 'include'}",
           f"-I{base / 'include' / 'torch' / 'csrc' / 'api' / 'include'}", "-Wno-deprecated-declarations",
           str(TORCH_SRC / "region_guard.cpp"), "-o", str(target) + ".tmp", f"-L{base / 'lib'}", "-ltorch_python",
           "-ltorch_cpu", "-ltorch", "-lc10", f"-Wl,-rpath,{base / 'lib'}"]
    if verbose:
        print(" ".join(cmd), file=sys.stderr)
    _run(cmd)
    os.replace(str(target) + ".tmp", target)
    return target


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
    print("built", ", ".join(LIBS))
