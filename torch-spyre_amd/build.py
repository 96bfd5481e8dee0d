"""In-tree build of the torch_spyre native pieces for MI355X (gfx950).

Produces, next to the Python sources so they travel with the tree:
  torch_spyre/lib/libspyre_hip.so   the C-ABI kernel library (hipcc, gfx950)
  torch_spyre/_C.<abi>.so           the PrivateUse1 backend extension (g++,
                                    ATen glue over the C-ABI)

Usage: python torch-spyre_amd/build.py [--only hip|aten] [-j N] [--incremental]
Every invocation recompiles everything (no stale objects survive a build).
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import sysconfig

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
INCLUDE = os.path.join(REPO, "include")
HIP_SRC = os.path.join(HERE, "csrc", "hip")
ATEN_SRC = os.path.join(HERE, "csrc", "aten")
PKG = os.path.join(HERE, "torch_spyre")
LIB_DIR = os.path.join(PKG, "lib")
BUILD_DIR = os.path.join(HERE, "_build")

ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")
OFFLOAD_ARCH = "gfx950"

HIP_FLAGS = [
    f"--offload-arch={OFFLOAD_ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    # Packed-fp32 VALU forms are kept out of every kernel.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
    f"-I{INCLUDE}",
    f"-I{HIP_SRC}",
]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(
        line for line in proc.stdout.splitlines()
        if "packed-fp32-ops" not in line  # host pass does not know the feature
    )
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")


def _torch_lib_dir() -> str:
    import torch

    return os.path.join(os.path.dirname(torch.__file__), "lib")


def _stale(obj: str, src: str, header_dirs: list[str]) -> bool:
    """True when obj is missing or older than src or any header under
    header_dirs."""
    if not os.path.exists(obj):
        return True
    t = os.path.getmtime(obj)
    deps = [src] + [os.path.join(d, f) for d in header_dirs for f in os.listdir(d)
                    if f.endswith((".h", ".hpp", ".cuh"))]
    return any(os.path.getmtime(p) > t for p in deps)


def build_hip(jobs: int, incremental: bool = False) -> str:
    objdir = os.path.join(BUILD_DIR, "hip")
    if not incremental:
        shutil.rmtree(objdir, ignore_errors=True)
    os.makedirs(objdir, exist_ok=True)
    os.makedirs(LIB_DIR, exist_ok=True)
    srcs = sorted(f for f in os.listdir(HIP_SRC) if f.endswith(".hip"))
    objs = [os.path.join(objdir, s[:-4] + ".o") for s in srcs]

    def compile_one(pair):
        src, obj = pair
        if incremental and not _stale(obj, os.path.join(HIP_SRC, src), [HIP_SRC, INCLUDE]):
            return obj
        _run([HIPCC, *HIP_FLAGS, "-c", os.path.join(HIP_SRC, src), "-o", obj])
        return obj

    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(compile_one, zip(srcs, objs)))
    out = os.path.join(LIB_DIR, "libspyre_hip.so")
    tmp = out + ".tmp"
    torch_lib = _torch_lib_dir()
    # Link against torch's bundled HIP runtime so a process that imports
    # torch carries exactly one HIP runtime.
    _run([HIPCC, f"--offload-arch={OFFLOAD_ARCH}", "-shared", "-fPIC", *objs, "-o", tmp,
          f"-L{torch_lib}", "-lamdhip64", f"-Wl,-rpath,{torch_lib}",
          "-Wl,-soname,libspyre_hip.so"])
    os.replace(tmp, out)
    return out


def build_aten(jobs: int, incremental: bool = False) -> str | None:
    if not os.path.isdir(ATEN_SRC):
        return None
    srcs = sorted(f for f in os.listdir(ATEN_SRC) if f.endswith(".cpp"))
    if not srcs:
        return None
    from torch.utils import cpp_extension

    objdir = os.path.join(BUILD_DIR, "aten")
    if not incremental:
        shutil.rmtree(objdir, ignore_errors=True)
    os.makedirs(objdir, exist_ok=True)
    py_inc = sysconfig.get_paths()["include"]
    incs = [f"-I{p}" for p in cpp_extension.include_paths()] + [
        f"-I{py_inc}", f"-I{INCLUDE}", f"-I{ATEN_SRC}", f"-I{ROCM}/include"]
    import torch

    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cflags = ["-O2", "-fPIC", "-std=c++17", "-fvisibility=hidden",
              f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-DTORCH_EXTENSION_NAME=_C",
              "-DTORCH_API_INCLUDE_EXTENSION_H", "-D__HIP_PLATFORM_AMD__=1",
              "-Wno-unused-parameter", "-Wno-deprecated-declarations", *incs]
    objs = [os.path.join(objdir, s[:-4] + ".o") for s in srcs]

    def compile_one(pair):
        src, obj = pair
        if incremental and not _stale(obj, os.path.join(ATEN_SRC, src), [ATEN_SRC, INCLUDE]):
            return obj
        _run(["g++", *cflags, "-c", os.path.join(ATEN_SRC, src), "-o", obj])
        return obj

    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(compile_one, zip(srcs, objs)))
    suffix = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
    out = os.path.join(PKG, "_C" + suffix)
    tmp = out + ".tmp"
    torch_lib = _torch_lib_dir()
    _run(["g++", "-shared", "-fPIC", *objs, "-o", tmp,
          f"-L{LIB_DIR}", "-lspyre_hip", "-Wl,-rpath,$ORIGIN/lib",
          f"-L{torch_lib}", "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python",
          "-lamdhip64", f"-Wl,-rpath,{torch_lib}"])
    os.replace(tmp, out)
    return out


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--only", choices=["hip", "aten"], default=None)
    ap.add_argument("-j", "--jobs", type=int, default=min(8, os.cpu_count() or 1))
    ap.add_argument("--incremental", action="store_true",
                    help="keep object files newer than their source and the headers")
    args = ap.parse_args(argv)
    if args.only in (None, "hip"):
        print("built", build_hip(args.jobs, args.incremental), flush=True)
    if args.only in (None, "aten"):
        out = build_aten(args.jobs, args.incremental)
        if out:
            print("built", out, flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
