"""Builds the bitcache gfx950 libraries in-tree.

  libbitcache_hip.so   the C ABI (include/bitcache.h): HIP kernels for gfx950
  _C.<abi>.so          PyTorch-ROCm extension over the C ABI (links the above)

Every HIP file is compiled with hipcc for --offload-arch=gfx950 only, with the
packed-fp32 instruction feature disabled.  Usage:  python -m bitcache_amd.build
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
import sysconfig

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
BUILD = os.path.join(HERE, "_build")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")
ARCH = "gfx950"

LIB = os.path.join(HERE, "libbitcache_hip.so")
EXT_SUFFIX = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
EXT = os.path.join(HERE, "_C" + EXT_SUFFIX)

HIP_SOURCES = ["encode.hip", "attention.hip", "attention_mfma.hip", "adaptive.hip", "convert.hip",
               "probe.hip", "abi.cpp"]
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I" + INCLUDE, "-I" + CSRC,
]


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError("build step failed:\n" + " ".join(cmd) + "\n" + out)
    return out


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, src + ".o")
    lang = [] if src.endswith(".hip") else ["-x", "hip"]
    _run([HIPCC] + HIP_FLAGS + lang + ["-c", os.path.join(CSRC, src), "-o", obj])
    return obj


def build_hip(jobs: int = 8) -> str:
    os.makedirs(BUILD, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, HIP_SOURCES))
    tmp = LIB + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp] + objs
         + [f"-Wl,-rpath,{ROCM}/lib", "-Wl,-soname,libbitcache_hip.so"])
    os.replace(tmp, LIB)
    return LIB


def build_ext() -> str:
    import torch
    from torch.utils import cpp_extension

    os.makedirs(BUILD, exist_ok=True)
    inc = cpp_extension.include_paths() + [sysconfig.get_paths()["include"], INCLUDE,
                                           os.path.join(ROCM, "include")]
    torch_lib = os.path.join(os.path.dirname(torch.__file__), "lib")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    tmp = EXT + ".tmp"
    cmd = (["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-w",
            "-D__HIP_PLATFORM_AMD__", "-DUSE_ROCM", "-DTORCH_EXTENSION_NAME=_C",
            "-DTORCH_API_INCLUDE_EXTENSION_H", f"-D_GLIBCXX_USE_CXX11_ABI={abi}"]
           + ["-I" + p for p in inc]
           + [os.path.join(CSRC, "torch_binding.cpp"), "-o", tmp,
              "-L" + HERE, "-lbitcache_hip",
              "-L" + torch_lib, "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip",
              "-ltorch_python",
              "-Wl,-rpath,$ORIGIN", "-Wl,-rpath," + torch_lib])
    _run(cmd)
    os.replace(tmp, EXT)
    return EXT


def build(jobs: int = 8) -> None:
    with cf.ThreadPoolExecutor(max_workers=2) as ex:
        f_hip = ex.submit(build_hip, jobs)
        f_hip.result()
        f_ext = ex.submit(build_ext)
        f_ext.result()


if __name__ == "__main__":
    build()
    print("built", LIB, EXT, file=sys.stderr)
