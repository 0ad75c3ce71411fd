"""In-tree build of the gfx950 library and the two drop-in extension modules.

    python -m santa_amd.build            # build everything
    python -m santa_amd.build --clean    # remove the built files

Products (git-ignored, shipped with the tree):
  santa_amd/libsanta_amd.so                 HIP kernels + the C ABI (include/santa_amd.h)
  santa_flash_batch_cuda/_C.<abi>.so        torch extension behind the drop-in package
  santa_prop_batch_cuda/_C.<abi>.so         torch extension behind the drop-in package

Native HIP sources are compiled with hipcc for gfx950 only; the extension
modules are plain host C++ compiled with g++ against the installed torch and
linked to libsanta_amd.so through an $ORIGIN-relative rpath.  There is no
hipify step and no CUDA code path.
"""
from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor
from typing import List

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
INCLUDE = os.path.join(REPO, "include")
BUILD_DIR = os.path.join(PKG_DIR, "_build")
LIB = os.path.join(PKG_DIR, "libsanta_amd.so")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")
ARCH = "gfx950"

HIP_SOURCES = ["santa_flash.hip", "santa_prop.hip", "santa_prop_gen.hip", "santa_runtime.hip"]
CXX_SOURCES = ["santa_common.cpp"]
EXTENSIONS = {"santa_flash_batch_cuda": "ext_flash.cpp", "santa_prop_batch_cuda": "ext_prop.cpp"}

# -ffp-contract=off: a*b+c is never fused unless written as fmaf(), so the
# sampled indices depend only on the association spelled out in the kernels.
# The packed-fp32 feature is switched off: v_pk_{add,mul,fma}_f32 are not used.
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off", "-fno-fast-math",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]


def _run(cmd: List[str]) -> None:
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"build step failed ({r.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out)


def ext_suffix() -> str:
    return sysconfig.get_config_var("EXT_SUFFIX") or ".so"


def ext_path(name: str) -> str:
    # The importable name is a package (repo root) whose __init__ imports
    # torch before the native module, so the process has exactly one HIP
    # runtime: torch's libamdhip64 (SONAME libamdhip64.so.7), which
    # libsanta_amd.so then binds to.
    return os.path.join(REPO, name, "_C" + ext_suffix())


def build_library() -> str:
    os.makedirs(BUILD_DIR, exist_ok=True)
    objs, cmds = [], []
    for src in HIP_SOURCES:
        if not os.path.exists(os.path.join(CSRC, src)):
            continue
        obj = os.path.join(BUILD_DIR, src + ".o")
        cmds.append([HIPCC, *HIP_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", "-c", os.path.join(CSRC, src), "-o", obj])
        objs.append(obj)
    for src in CXX_SOURCES:
        obj = os.path.join(BUILD_DIR, src + ".o")
        cmds.append([HIPCC, "-O2", "-std=c++17", "-fPIC", "-D__HIP_PLATFORM_AMD__", f"-I{INCLUDE}", f"-I{CSRC}",
                     "-c", os.path.join(CSRC, src), "-o", obj])
        objs.append(obj)
    with ThreadPoolExecutor(max_workers=min(8, len(cmds))) as ex:
        list(ex.map(_run, cmds))
    tmp = LIB + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs, "-Wl,-soname,libsanta_amd.so"])
    os.replace(tmp, LIB)
    return LIB


def build_extension(name: str, src: str) -> str:
    import torch
    from torch.utils import cpp_extension

    torch_dir = os.path.dirname(torch.__file__)
    incs = cpp_extension.include_paths() + [os.path.join(ROCM, "include"), INCLUDE, CSRC,
                                            sysconfig.get_paths()["include"]]
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    out = ext_path(name)
    tmp = out + ".tmp"
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-w",
           f"-D_GLIBCXX_USE_CXX11_ABI={abi}", f"-DTORCH_EXTENSION_NAME=_C", "-DTORCH_API_INCLUDE_EXTENSION_H",
           "-DUSE_ROCM=1", "-D__HIP_PLATFORM_AMD__=1",
           *[f"-I{i}" for i in incs], os.path.join(CSRC, src), "-o", tmp,
           f"-L{os.path.join(torch_dir, 'lib')}", f"-L{PKG_DIR}",
           "-lsanta_amd", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip", "-ltorch_python",
           "-Wl,-rpath,$ORIGIN/../santa_amd", f"-Wl,-rpath,{os.path.join(torch_dir, 'lib')}"]
    _run(cmd)
    os.replace(tmp, out)
    return out


def build_all(verbose: bool = True) -> None:
    lib = build_library()
    if verbose:
        print(f"[santa_amd.build] {lib}")
    todo = [(n, s) for n, s in EXTENSIONS.items() if os.path.exists(os.path.join(CSRC, s))]
    with ThreadPoolExecutor(max_workers=len(todo) or 1) as ex:
        for path in ex.map(lambda ns: build_extension(*ns), todo):
            if verbose:
                print(f"[santa_amd.build] {path}")


def clean() -> None:
    shutil.rmtree(BUILD_DIR, ignore_errors=True)
    for p in [LIB] + [ext_path(n) for n in EXTENSIONS]:
        if os.path.exists(p):
            os.remove(p)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--clean", action="store_true")
    args = ap.parse_args(argv)
    if args.clean:
        clean()
        return 0
    build_all()
    return 0


if __name__ == "__main__":
    sys.exit(main())
