"""Write golden vectors from the reference's own CPU extension.

Runs philtorch's CPU operators, compiled from /root/reference/philtorch/csrc by
oracle/build_ref.py into oracle/_ref/ref_C.so, on small seeded inputs and
stores inputs and outputs in tests/golden/ref_vectors.npz.  Only data is
committed; the reference itself never travels with the repository.

    python oracle/build_ref.py && python tests/golden/make_golden.py
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, REPO)

from oracle import ref_runner  # noqa: E402


def cases():
    g = np.random.default_rng(20261201)
    out = []
    for dt in (np.float32, np.float64, np.complex64, np.complex128):
        cplx = np.dtype(dt).kind == "c"

        def rnd(*shape):
            v = g.standard_normal(shape)
            if cplx:
                v = v + 1j * g.standard_normal(shape)
            return v.astype(dt)

        def coef(*shape):
            v = g.uniform(-0.95, 0.95, shape)
            if cplx:
                v = v * np.exp(1j * g.uniform(0, np.pi, shape))
            return v.astype(dt)

        B, T = 3, 37
        # recurN with M = 1 (LPV scalar), batched and shared coefficient
        out.append(("recurN", coef(B, T, 1, 1), rnd(B, 1), rnd(B, T, 1)))
        out.append(("recurN", coef(T, 1, 1), rnd(B, 1), rnd(B, T, 1)))
        # recurN with M = 2 (the recur2 math)
        out.append(("recurN", 0.6 * coef(B, T, 2, 2), rnd(B, 2), rnd(B, T, 2)))
        out.append(("recurN", 0.6 * coef(T, 2, 2), rnd(B, 2), rnd(B, T, 2)))
        # LTI scalar: per-row and shared a
        out.append(("lti_recur", coef(B), rnd(B), rnd(B, T)))
        out.append(("lti_recur", coef(1), rnd(B), rnd(B, T)))
        # LTI 2x2: per-row and shared A
        out.append(("lti_recurN", 0.6 * coef(B, 2, 2), rnd(B, 2), rnd(B, T, 2)))
        out.append(("lti_recurN", 0.6 * coef(2, 2), rnd(B, 2), rnd(B, T, 2)))
    # README Fibonacci known answer through lti_recurN in int64
    x = np.zeros((1, 10, 2), np.int64)
    x[0, 0, 0] = 1
    out.append(("lti_recurN", np.array([[1, 1], [1, 0]], np.int64), np.zeros((1, 2), np.int64), x))
    # orders 3 and 4 (recurN / lti_recurN beyond 2x2), batched and shared
    # coefficients; a generator of their own keeps the cases above unchanged
    g3 = np.random.default_rng(20261202)
    for dt in (np.float32, np.float64, np.complex64, np.complex128):
        cplx = np.dtype(dt).kind == "c"

        def rnd3(*shape):
            v = g3.standard_normal(shape)
            if cplx:
                v = v + 1j * g3.standard_normal(shape)
            return v.astype(dt)

        def coef3(M, *shape):
            # entries below 0.9/M in modulus: every row sums below 0.9, a contraction
            v = g3.uniform(-0.9 / M, 0.9 / M, shape)
            if cplx:
                v = v * np.exp(1j * g3.uniform(0, np.pi, shape))
            return v.astype(dt)

        B, T = 3, 37
        for M in (3, 4):
            out.append(("recurN", coef3(M, B, T, M, M), rnd3(B, M), rnd3(B, T, M)))
            out.append(("recurN", coef3(M, T, M, M), rnd3(B, M), rnd3(B, T, M)))
            out.append(("lti_recurN", coef3(M, B, M, M), rnd3(B, M), rnd3(B, T, M)))
            out.append(("lti_recurN", coef3(M, M, M), rnd3(B, M), rnd3(B, T, M)))
    # half and bfloat16: the reference's CPU loops run in those types, rounding
    # after every operation; bfloat16 arrays are stored as their 16-bit
    # patterns (uint16) with a dtype tag
    import torch

    g16 = np.random.default_rng(20261203)
    for dt in ("float16", "bfloat16"):

        def cast(v, dt=dt):
            t = torch.from_numpy(np.ascontiguousarray(v, dtype=np.float32)).to(getattr(torch, dt))
            return t.view(torch.uint16).numpy() if dt == "bfloat16" else t.numpy()

        def rnd16(*shape):
            return cast(g16.standard_normal(shape))

        def coef16(*shape):
            return cast(g16.uniform(-0.95, 0.95, shape))

        B, T = 3, 37
        out.append(("recurN", coef16(B, T, 1, 1), rnd16(B, 1), rnd16(B, T, 1), dt))
        out.append(("recurN", coef16(T, 1, 1), rnd16(B, 1), rnd16(B, T, 1), dt))
        out.append(("recurN", cast(0.6 * g16.uniform(-0.95, 0.95, (B, T, 2, 2))), rnd16(B, 2), rnd16(B, T, 2), dt))
        out.append(("recurN", cast(0.6 * g16.uniform(-0.95, 0.95, (T, 2, 2))), rnd16(B, 2), rnd16(B, T, 2), dt))
        out.append(("lti_recur", coef16(B), rnd16(B), rnd16(B, T), dt))
        out.append(("lti_recur", coef16(1), rnd16(B), rnd16(B, T), dt))
        out.append(("lti_recurN", cast(0.6 * g16.uniform(-0.95, 0.95, (B, 2, 2))), rnd16(B, 2), rnd16(B, T, 2), dt))
        out.append(("lti_recurN", cast(0.6 * g16.uniform(-0.95, 0.95, (2, 2))), rnd16(B, 2), rnd16(B, T, 2), dt))
    return out


def main() -> None:
    arrays = {}
    for i, case in enumerate(cases()):
        op, A, zi, x = case[:4]
        dt = case[4] if len(case) > 4 else ""
        y = ref_runner.run(op, A, zi, x, dt)
        arrays[f"{i}_op"] = np.array(op)
        arrays[f"{i}_A"], arrays[f"{i}_zi"], arrays[f"{i}_x"], arrays[f"{i}_y"] = A, zi, x, y
        if dt:
            arrays[f"{i}_dt"] = np.array(dt)
    path = os.path.join(HERE, "ref_vectors.npz")
    np.savez_compressed(path, **arrays)
    print(f"wrote {sum(1 for k in arrays if k.endswith('_op'))} cases to {path}")


if __name__ == "__main__":
    main()
