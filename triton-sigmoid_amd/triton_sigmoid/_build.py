"""Builds libsigattn.so (the gfx950 kernels + C ABI) in-tree with hipcc, and
the C++ autograd node of the eager public APIs (_sigattn_autograd) with g++.

Every HIP source is compiled for gfx950 only, with packed-fp32 instruction
selection disabled (``-Xclang -target-feature -Xclang -packed-fp32-ops``), and
linked into ``triton_sigmoid/libsigattn.so`` next to this file.  The autograd
node (csrc/torch_autograd.cpp) is host-only C++ against torch's headers and
libraries; it calls libsigattn through entry point addresses handed over at
run time, so it does not link the kernel library.
"""

from __future__ import annotations

import concurrent.futures as _cf
import os
import shutil
import subprocess
import sysconfig
import warnings
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
ROOT = PKG_DIR.parent
CSRC = ROOT / "csrc"
INCLUDE = ROOT.parent / "include"
LIB_PATH = PKG_DIR / "libsigattn.so"
BUILD_DIR = ROOT / "_build"

SOURCES = ["fwd.hip", "bwd.hip", "decode.hip", "f32.hip", "generic.hip", "capi.cpp"]
ARCH = "gfx950"
AUTOGRAD_SOURCE = "torch_autograd.cpp"
AUTOGRAD_NAME = "_sigattn_autograd"


def hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(exe):
        raise RuntimeError("hipcc not found; the ROCm toolchain is required to build libsigattn.so")
    return exe


def compile_flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        f"-I{CSRC}",
        f"-I{INCLUDE}",
    ]


def _compile(src: Path, obj: Path, defines: tuple = ()) -> None:
    lang = ["-x", "hip"] if src.suffix == ".cpp" else []
    cmd = [hipcc(), *compile_flags(), *defines, *lang, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stdout}\n{res.stderr}")


def autograd_path() -> Path:
    return PKG_DIR / (AUTOGRAD_NAME + sysconfig.get_config_var("EXT_SUFFIX"))


def build_autograd(out: Path | None = None) -> Path:
    """Compiles the C++ autograd node into the package (or `out`)."""
    import torch
    from torch.utils import cpp_extension

    target = Path(out) if out is not None else autograd_path()
    tmp = target.with_name(target.name + ".tmp")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = [shutil.which("g++") or "g++", "-O2", "-std=c++17", "-fPIC", "-shared",
           f"-D_GLIBCXX_USE_CXX11_ABI={abi}", f"-DTORCH_EXTENSION_NAME={AUTOGRAD_NAME}",
           "-DTORCH_API_INCLUDE_EXTENSION_H", "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
           *(f"-I{p}" for p in cpp_extension.include_paths()),
           f"-I{sysconfig.get_paths()['include']}", f"-I{_rocm_include()}",
           str(CSRC / AUTOGRAD_SOURCE), "-o", str(tmp),
           *(f"-L{p}" for p in cpp_extension.library_paths()),
           "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_python", "-lamdhip64"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"g++ failed for {AUTOGRAD_SOURCE}:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, target)
    return target


def _rocm_include() -> str:
    return str(Path(os.path.realpath(hipcc())).parent.parent / "include")


def build(verbose: bool = False, jobs: int = 4, defines: tuple = (), out: Path | None = None) -> Path:
    """Compiles every source and links LIB_PATH (or `out`).  Always rebuilds.
    The default build also compiles the C++ autograd node (build_autograd).

    `defines` are extra -D options for the tile-configuration macros of the
    kernel sources (e.g. "-DSIGATTN_FWD_D64_STAGES=4"); a build with them
    goes to `out` (its objects to a folder of their own), and _capi loads it
    when the environment variable SIGATTN_LIBRARY names it."""
    defines = tuple(defines)
    if defines and out is None:
        raise ValueError("a build with extra defines needs its own output path")
    lib = Path(out) if out is not None else LIB_PATH
    bdir = BUILD_DIR if not defines else BUILD_DIR / ("variant_" + lib.stem)
    bdir.mkdir(parents=True, exist_ok=True)
    objs = [bdir / (Path(s).stem + ".o") for s in SOURCES]
    with _cf.ThreadPoolExecutor(max_workers=jobs + 1) as ex:
        futs = [ex.submit(_compile, CSRC / s, o, defines) for s, o in zip(SOURCES, objs)]
        node = ex.submit(build_autograd) if out is None else None
        for f in futs:
            f.result()
        if node is not None:
            # The kernel library does not depend on the autograd node: without
            # g++ or torch's headers the Python nodes serve the eager APIs
            # (_capi.autograd_node warns and falls back when the import fails),
            # so a failed node build is a warning and the library still links.
            try:
                node.result()
            except Exception as e:  # noqa: BLE001 -- any failure of the optional node
                stale = autograd_path()
                if stale.exists():
                    stale.unlink()  # an older node built against other sources must not load
                warnings.warn(f"C++ autograd node not built ({e}); the Python autograd nodes will serve")
    tmp = lib.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, lib)
    if verbose:
        print(f"built {lib}" + (f" and {autograd_path()}" if out is None else ""))
    return lib


if __name__ == "__main__":
    import argparse

    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--out", type=Path, help="output library (required with -D options)")
    args, defines = ap.parse_known_args()
    if any(not d.startswith("-D") for d in defines):
        ap.error(f"unknown arguments {defines}")
    build(verbose=True, defines=tuple(defines), out=args.out)
