"""In-tree build of philtorch_amd's native code for gfx950.

Two shared objects, both written next to this file so that they travel with
the repository tree:

* ``libphilscan.so`` — the HIP kernels and their C ABI (include/philscan.h),
  compiled by hipcc for gfx950 only from units compiled in parallel
  (fixed-order and order-M entry points, the order-3 and order-4 kernels,
  the fused second-order-section cascade, the fused single-input
  single-output LTI state space with filtfilt, the LPV state space, and the
  streaming probe the bench times beside the scans).
  It has no torch dependency.
* ``_C.so`` — the torch.library operator layer (csrc/torch_ops.cpp), host C++
  linked against libtorch and libphilscan (found through ``$ORIGIN``).

No hipify step, no JIT cache: ``python -m philtorch_amd._build`` or
``__graft_entry__.build()`` runs the compiles in parallel.
"""
from __future__ import annotations

import os
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
REPO = os.path.dirname(HERE)
INCLUDE = os.path.join(REPO, "include")
ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# hipcc-only flags: no packed-FP32 instructions are generated (a correctness
# guard for this hardware pool); code object v5 loads under every ROCm 6/7
# runtime; the atomic optimizer is off: every atomic here is issued by one
# lane already, and the optimizer's rewrite waits for the result at once,
# which would put the tile claim's round trip in front of the tile's loads.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-mcode-object-version=5",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-atomic-optimizer-strategy=None",
    "-Wall", "-Wno-unused-local-typedef", "-Wno-unknown-pragmas",
]

KERNEL_LIB = os.path.join(HERE, "libphilscan.so")
OPS_LIB = os.path.join(HERE, "_C.so")


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(
        line for line in proc.stdout.splitlines() if "packed-fp32-ops" not in line or "error" in line
    )
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}):\n{' '.join(cmd)}\n{out}")
    if verbose and out.strip():
        print(out, flush=True)


# (source, extra flags, object): the fixed-order and order-M entry points,
# the generic BlockN kernels once per order, the SOS cascade (and filtfilt),
# and the single-input single-output state space
KERNEL_UNITS = (
    ("phs_capi.hip", [], "phs_capi.o"),
    ("phs_capi_n.hip", [], "phs_capi_n.o"),
    ("phs_blockn.hip", ["-DPHS_BLOCKN_ORDER=3"], "phs_blockn3.o"),
    ("phs_blockn.hip", ["-DPHS_BLOCKN_ORDER=4"], "phs_blockn4.o"),
    ("phs_sos.hip", [], "phs_sos.o"),
    ("phs_ss.hip", [], "phs_ss.o"),
    ("phs_lpvss.hip", [], "phs_lpvss.o"),
    ("phs_mimo.hip", [], "phs_mimo.o"),
    ("phs_probe.hip", [], "phs_probe.o"),
)


def _kernel_cmds() -> tuple[list[list[str]], list[str]]:
    """(per-unit compile commands, link command) of libphilscan."""
    objs = [os.path.join(HERE, o) for _, _, o in KERNEL_UNITS]
    compiles = [[HIPCC, *HIP_FLAGS, *flags, "-c", os.path.join(CSRC, src), "-o", o]
                for (src, flags, _), o in zip(KERNEL_UNITS, objs)]
    link = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-Wl,-soname,libphilscan.so", *objs, "-o", KERNEL_LIB + ".tmp"]
    return compiles, link


def _ops_cmds() -> tuple[list[str], list[str]]:
    """(compile, link) commands of the torch.library layer."""
    import torch
    from torch.utils import cpp_extension

    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    incs = cpp_extension.include_paths() + [sysconfig.get_paths()["include"], INCLUDE]
    libdirs = cpp_extension.library_paths()
    obj = OPS_LIB + ".o"
    compile_cmd = [
        "g++", "-O2", "-std=c++17", "-fPIC", "-w", "-c",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
        *[f"-I{i}" for i in incs], "-I/opt/rocm/include",
        os.path.join(CSRC, "torch_ops.cpp"), "-o", obj,
    ]
    link_cmd = [
        "g++", "-shared", obj, "-o", OPS_LIB + ".tmp",
        *[f"-L{d}" for d in libdirs], f"-L{HERE}",
        "-Wl,-rpath,$ORIGIN", *[f"-Wl,-rpath,{d}" for d in libdirs],
        "-lphilscan", "-lc10", "-lc10_hip", "-ltorch_cpu", "-ltorch_hip", "-ltorch",
    ]
    return compile_cmd, link_cmd


def build(verbose: bool = False) -> list[str]:
    """Compile both libraries; returns their paths.  Always recompiles."""
    compile_cmd, link_cmd = _ops_cmds()
    kernel_compiles, kernel_link = _kernel_cmds()
    with ThreadPoolExecutor(max_workers=len(kernel_compiles) + 1) as ex:
        futs = [ex.submit(_run, c, verbose) for c in kernel_compiles] + [ex.submit(_run, compile_cmd, verbose)]
        for f in futs:
            f.result()
    _run(kernel_link, verbose)
    for c in kernel_compiles:
        os.remove(c[-1])
    os.replace(KERNEL_LIB + ".tmp", KERNEL_LIB)
    _run(link_cmd, verbose)
    os.replace(OPS_LIB + ".tmp", OPS_LIB)
    os.remove(OPS_LIB + ".o")
    return [KERNEL_LIB, OPS_LIB]


if __name__ == "__main__":
    for p in build(verbose="-v" in sys.argv):
        print(p)
