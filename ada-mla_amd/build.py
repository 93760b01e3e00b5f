"""Builds the MLA decode library in-tree.

  ada_mla/libmla_mi355x.so  the HIP kernels + C ABI (include/mla_mi355x.h),
                            hipcc --offload-arch=gfx950
  ada_mla/_C*.so            the PyTorch extension (csrc/mla_api.cpp), g++,
                            linked against libmla_mi355x.so (rpath $ORIGIN)

The .hip sources are compiled by hipcc directly (not through
torch.utils.cpp_extension, which would run hipify on them). Objects go to
ada-mla_amd/_build/ (git-ignored). Usage: python ada-mla_amd/build.py [--lib-only | --timeline]
(--timeline: only the instrumented ada_mla/libmla_mi355x_timeline.so, see build_lib)
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import sysconfig

PKG_ROOT = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(PKG_ROOT)
CSRC = os.path.join(PKG_ROOT, "csrc")
OUT_DIR = os.path.join(PKG_ROOT, "ada_mla")
BUILD = os.path.join(PKG_ROOT, "_build")
INCLUDE = os.path.join(REPO, "include")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

HIP_SOURCES = ["mla_splitkv_fp16.hip", "mla_splitkv_fp32.hip", "mla_combine.hip", "mla_capi.hip",
               "mla_block.hip"]
LIB_NAME = "libmla_mi355x.so"
TIMELINE_LIB_NAME = "libmla_mi355x_timeline.so"

HIPCC_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    "-mcode-object-version=5",
    # packed fp32 VALU ops are kept out of the generated code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
    # the first 16 dwords of every kernel's arguments arrive in SGPRs at wave
    # launch instead of through a kernel-argument fetch at the kernel's start
    # (same box, against none: N = 4096 11.55 -> 11.24 us per call, n_h = 16
    # 16.31 -> 15.91 us; preloading the combine's arguments alone gained
    # nothing measurable)
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    f"-I{INCLUDE}", f"-I{CSRC}",
]


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines()
                    if "packed-fp32-ops' is not a recognized feature" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{out}")
    return out


def build_lib(jobs: int = 4, timeline: bool = False) -> str:
    """The library; with timeline=True the instrumented copy
    ada_mla/libmla_mi355x_timeline.so (-DMLA_TIMELINE: the split kernel records
    per-workgroup phase stamps, read by ada-mla_amd/timeline.py), which
    nothing else loads."""
    build_dir = os.path.join(BUILD, "timeline") if timeline else BUILD
    os.makedirs(build_dir, exist_ok=True)
    hipcc = os.path.join(ROCM, "bin", "hipcc")
    objs = []
    cmds = []
    extra = ["-DMLA_TIMELINE"] if timeline else []
    for src in HIP_SOURCES:
        obj = os.path.join(build_dir, src.replace(".hip", ".o"))
        objs.append(obj)
        cmds.append([hipcc, *HIPCC_FLAGS, *extra, "-c", os.path.join(CSRC, src), "-o", obj])
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        for out in ex.map(_run, cmds):
            if out.strip():
                print(out)
    lib = os.path.join(OUT_DIR, TIMELINE_LIB_NAME if timeline else LIB_NAME)
    tmp = lib + ".tmp"
    _run([hipcc, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp])
    os.replace(tmp, lib)
    return lib


def build_ext() -> str:
    import torch.utils.cpp_extension as ce
    import torch
    ext_suffix = sysconfig.get_config_var("EXT_SUFFIX")
    target = os.path.join(OUT_DIR, "_C" + ext_suffix)
    obj = os.path.join(BUILD, "mla_api.o")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    incs = [*ce.include_paths(), sysconfig.get_paths()["include"], os.path.join(ROCM, "include"), INCLUDE]
    _run(["g++", "-O2", "-std=c++17", "-fPIC", "-c", os.path.join(CSRC, "mla_api.cpp"), "-o", obj,
          "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", "-DTORCH_EXTENSION_NAME=_C",
          "-DTORCH_API_INCLUDE_EXTENSION_H", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
          "-Wno-deprecated-declarations", *[f"-I{p}" for p in incs]])
    libdirs = ce.library_paths()
    tmp = target + ".tmp"
    _run(["g++", "-shared", "-o", tmp, obj, *[f"-L{p}" for p in libdirs], f"-L{OUT_DIR}",
          "-lmla_mi355x", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_python",
          "-Wl,-rpath,$ORIGIN"])
    os.replace(tmp, target)
    return target


def build(lib_only: bool = False, timeline: bool = False) -> None:
    if timeline:
        print(f"built {os.path.relpath(build_lib(timeline=True), REPO)}")
        return
    lib = build_lib()
    print(f"built {os.path.relpath(lib, REPO)}")
    if not lib_only:
        ext = build_ext()
        print(f"built {os.path.relpath(ext, REPO)}")


if __name__ == "__main__":
    build(lib_only="--lib-only" in sys.argv, timeline="--timeline" in sys.argv)
