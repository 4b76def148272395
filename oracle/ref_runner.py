"""Run the reference's own CPU operators (oracle/_ref/ref_C.so) in isolation.

Test infrastructure only.  ref_C.so owns TORCH_LIBRARY(philtorch), so it is
loaded in a fresh child process (never next to philtorch_amd's _C.so):

    python -m oracle.ref_runner IN.npz OUT.npz

IN.npz holds `op` (recurN | lti_recurN | lti_recur) and arrays A, zi, x;
OUT.npz receives y computed by torch.ops.philtorch.<op> on the CPU.  With
`dt` = "bfloat16" (numpy has no such dtype) the arrays in and out are the
values' 16-bit patterns as uint16.
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REF_LIB = os.path.join(HERE, "_ref", "ref_C.so")


def main(inp: str, out: str) -> None:
    import torch

    torch.ops.load_library(REF_LIB)
    data = np.load(inp)
    op = str(data["op"])
    bf16 = "dt" in data.files and str(data["dt"]) == "bfloat16"
    A, zi, x = (torch.from_numpy(np.ascontiguousarray(data[k])) for k in ("A", "zi", "x"))
    if bf16:
        A, zi, x = (v.view(torch.bfloat16) for v in (A, zi, x))
    y = getattr(torch.ops.philtorch, op)(A, zi, x)
    np.savez(out, y=(y.view(torch.uint16) if bf16 else y).numpy())


def run(op: str, A, zi, x, dt: str = "") -> np.ndarray:
    """Call the reference op in a child process and return its output
    (dt="bfloat16": arrays in and out are uint16 bit patterns)."""
    import subprocess
    import tempfile

    with tempfile.TemporaryDirectory() as d:
        fi, fo = os.path.join(d, "in.npz"), os.path.join(d, "out.npz")
        np.savez(fi, op=np.array(op), A=A, zi=zi, x=x, dt=np.array(dt))
        env = dict(os.environ, PYTHONPATH=os.path.dirname(HERE))
        subprocess.run([sys.executable, "-m", "oracle.ref_runner", fi, fo], check=True, env=env,
                       cwd=os.path.dirname(HERE))
        return np.load(fo)["y"]


if __name__ == "__main__":
    main(sys.argv[1], sys.argv[2])
