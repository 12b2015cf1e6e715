#!/usr/bin/env python3
"""Writes tests/golden/dot2c_bf16.npz: gfx950 v_dot2c_f32_bf16 outputs on one MI355X, for the
oracle's model of the instruction (oracle/fleet_oracle.c, dot2_hw; tests/test_dot2_model.py).

    python tests/golden/make_dot2_fixture.py OUT.npz      (on a GPU box; libfleet_probe.so built)

Cases: crafted sums that separate candidate orders (two half-ulp terms on 1, a tiny product after
a cancellation, the accumulator just below and above the products' grid, products far apart,
subnormal bf16 inputs) and random cases at GEMV scales and with wide exponent spreads. A = pairs
of bf16 (element 0 in bits 0..15), B likewise, C the accumulators, D the instruction's results."""
import ctypes
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path[:0] = [str(ROOT), str(ROOT / "fleet-amd-task_amd")]
from fleet import runtime as R  # noqa: E402


def bf(x):
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint32)


def cases(seed=7):
    rng = np.random.default_rng(seed)
    a0, a1, b0, b1, c = [], [], [], [], []

    def add(x0, x1, y0, y1, acc):
        a0.append(bf(x0)); a1.append(bf(x1)); b0.append(bf(y0)); b1.append(bf(y1)); c.append(np.float32(acc))

    add(2.0 ** -12, 2.0 ** -12, 2.0 ** -12, 2.0 ** -12, 1.0)       # 1 + 2^-24 + 2^-24
    add(1.0, 2.0 ** -30, -1.0, 1.5, 1.0)                             # 1 - 1 + 1.5 2^-30
    for j in range(20, 61):
        for s in (1.0, -1.0):
            add(1.0, 0.0, 1.0, 0.0, s * 2.0 ** -j)                   # accumulator below the grid
            add(1.0, 1.0, 1.0, s * 2.0 ** -j, 0.0)                   # second product below
            add(1.0, 1.0, -1.0, s * 2.0 ** -j, 1.0 + 2.0 ** -23)     # cancellation, then the tail
    for j in range(1, 48):
        add(1.0, 1.0, 1.0, 1.0, 2.0 ** j)                            # accumulator above the products
        add(1.5, -1.25, 1.0, 2.0 ** -j, -(2.0 ** (j // 2)))
    for e in range(-133, -125):
        add(2.0 ** e, 2.0 ** (e + 3), 1.0, 3.0, 2.0 ** -150 * 3)    # subnormal bf16 inputs
    n = 4096
    w = rng.normal(0, 0.02, (n, 2)) * np.exp2(rng.integers(-8, 8, (n, 2)))
    x = rng.normal(0, 1, (n, 2)) * np.exp2(rng.integers(-12, 12, (n, 2)))
    acc = rng.normal(0, 1, n) * np.exp2(rng.integers(-30, 30, n))
    for i in range(n):
        add(w[i, 0], w[i, 1], x[i, 0], x[i, 1], acc[i])
    A = (np.array(a0) | (np.array(a1) << 16)).astype(np.uint32)
    B = (np.array(b0) | (np.array(b1) << 16)).astype(np.uint32)
    return A, B, np.array(c, np.float32)


def main():
    out = sys.argv[1] if len(sys.argv) > 1 else str(Path(__file__).with_name("dot2c_bf16.npz"))
    rt = R.Runtime(0)
    L = ctypes.CDLL(str(ROOT / "fleet-amd-task_amd" / "lib" / "libfleet_probe.so"))
    u32p, f32p = ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(ctypes.c_float)
    L.fxp_dot2.argtypes = [u32p, u32p, f32p, f32p, ctypes.c_int]
    A, B, C = cases()
    D = np.zeros(len(A), np.float32)
    assert L.fxp_dot2(A.ctypes.data_as(u32p), B.ctypes.data_as(u32p), C.ctypes.data_as(f32p),
                      D.ctypes.data_as(f32p), len(A)) == 0
    np.savez_compressed(out, A=A, B=B, C=C, D=D)
    print(f"wrote {out}: {len(A)} cases", flush=True)
    rt.close()


if __name__ == "__main__":
    main()
