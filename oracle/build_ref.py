"""Compile the reference's CPU extension from its own sources into oracle/_ref/.

Test infrastructure only.  The four CPU files of philtorch/csrc
(host_recur2.cpp, host_recurN.cpp, host_lti_recur.cpp, host_lti_recurN.cpp)
include nothing but torch headers, so g++ builds them directly where they lie
under the reference tree; nothing is copied into this repository.  The result,
oracle/_ref/ref_C.so, owns `TORCH_LIBRARY(philtorch)` exactly as the
reference's `_C` does, so it must never be loaded into a process that also
loads philtorch_amd's `_C.so` (duplicate namespace definitions abort).
oracle/ref_runner.py loads it in a child process.

The CUDA sources are not built (no CUDA toolchain here).
"""
import argparse
import os
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor

SOURCES = ["host_recur2.cpp", "host_recurN.cpp", "host_lti_recur.cpp", "host_lti_recurN.cpp"]


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--ref", default="/root/reference")
    ap.add_argument("--out", default=os.path.join(os.path.dirname(os.path.abspath(__file__)), "_ref"))
    args = ap.parse_args()
    csrc = os.path.join(args.ref, "philtorch", "csrc")
    if not os.path.isdir(csrc):
        print(f"reference sources not found at {csrc}; skipping", file=sys.stderr)
        return 0
    import torch
    from torch.utils import cpp_extension

    os.makedirs(args.out, exist_ok=True)
    incs = cpp_extension.include_paths() + [sysconfig.get_paths()["include"]]
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cflags = ["-O2", "-fPIC", "-fopenmp", "-std=c++17", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
              "-DTORCH_EXTENSION_NAME=_C", "-w"] + [f"-I{i}" for i in incs]

    def compile_one(src):
        obj = os.path.join(args.out, src.replace(".cpp", ".o"))
        cmd = ["g++", *cflags, "-c", os.path.join(csrc, src), "-o", obj]
        subprocess.run(cmd, check=True)
        return obj

    with ThreadPoolExecutor(max_workers=4) as ex:
        objs = list(ex.map(compile_one, SOURCES))
    libdirs = cpp_extension.library_paths()
    so = os.path.join(args.out, "ref_C.so")
    cmd = ["g++", "-shared", "-fopenmp", *objs, "-o", so] + [f"-L{d}" for d in libdirs] + \
          [f"-Wl,-rpath,{d}" for d in libdirs] + ["-lc10", "-ltorch_cpu", "-ltorch"]
    subprocess.run(cmd, check=True)
    for o in objs:
        os.remove(o)
    print(so)
    return 0


if __name__ == "__main__":
    sys.exit(main())
