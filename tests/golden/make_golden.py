"""Write tests/golden/fakequant_kat.npz: known-answer vectors for the three QAT fake-quants.

Inputs are the ones the reference's own unit test draws (tests/test_parity.py:318-331):
``np.random.default_rng(3)``; a [256, 64] log-normal-scaled normal matrix, then the
exact e4m3/e2m1 midpoint vector tiled to [2, 64] and scaled by 2**U{-8..8} per row.

Expected outputs are computed WITHOUT the oracle's bit tricks or threshold tables:
scales come from ``math.frexp`` and every rounding is a brute-force nearest search
over the full decoded e4m3fn / e2m1 code tables, ties to the even code. That makes
the fixture an independent check of ``oracle/cpu_ref.py``'s fake-quants
(fakequant.py:47-119 and kernel.py:22-37, 40-204 are the semantics restated).

Run:  python tests/golden/make_golden.py
"""

from __future__ import annotations

import math
import os

import numpy as np

F32 = np.float32
HERE = os.path.dirname(os.path.abspath(__file__))


def fp4_tie_inputs():
    """Blocks whose amax is exactly 6 * 2^e, so x / scale lands exactly on every e2m1
    rounding midpoint (the reference's own midpoint vector never reaches them at fp4:
    each of its 32-blocks holds 448, which scales the rest to ~0)."""
    mids = [0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0]
    row = [6.0] + mids + [-m for m in mids] + [0.5, 1.0, 1.5, 2.0, 3.0, 4.0, -6.0, 0.0,
                                              0.1, 5.9, 0.74, 0.76, 2.49, 2.51, 4.99, 5.01, 3.49]
    row = np.array(row[:32], dtype=F32)
    e = np.arange(-6, 7, dtype=F32)[:, None]
    return (row[None, :] * 2.0 ** e).astype(F32)


def reference_inputs():
    """The reference test's two input arrays (tests/test_parity.py:323-331)."""
    rng = np.random.default_rng(3)
    a = (rng.standard_normal((256, 64)) * np.exp(rng.standard_normal((256, 1)))).astype(F32)
    b = (np.array([0.033203125, -0.033203125, 0.25, 0.75, 1.25, 1.75, 2.5, 3.5,
                   5.0, -5.0, 448.0, 6.0, 1e-9, 0.0, -0.0, 2.0] * 8, dtype=F32)
         .reshape(2, 64) * 2.0 ** rng.integers(-8, 9, size=(2, 1)).astype(F32))
    return [a, b.astype(F32)]


def e4m3_table():
    """All finite non-negative e4m3fn values in code order (code 0x7F is NaN)."""
    vals = []
    for code in range(0x7F):
        e, m = code >> 3, code & 7
        vals.append(m * 2.0 ** -9 if e == 0 else (1 + m / 8) * 2.0 ** (e - 7))
    return np.array(vals, dtype=np.float64)


E4M3 = e4m3_table()
E2M1 = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], dtype=np.float64)


def nearest_even(v: float, table: np.ndarray) -> float:
    """Nearest table magnitude to |v|, ties to the even code, sign of v kept."""
    a = abs(float(v))
    d = np.abs(table - a)
    best = d.min()
    codes = np.nonzero(d == best)[0]
    code = codes[0] if len(codes) == 1 else [c for c in codes if c % 2 == 0][0]
    return math.copysign(float(table[code]), float(v))


def pow2_ceil(r: float) -> float:
    """2**ceil(log2 r) for positive normal r via frexp (r = f * 2**e, f in [0.5, 1))."""
    f, e = math.frexp(r)
    return 2.0 ** (e - 1) if f == 0.5 else 2.0 ** e


def f32(x) -> float:
    return float(np.float32(x))


def fq_fp8_ue8m0(x, block=32):
    out = np.empty_like(x)
    for i in range(x.shape[0]):
        for j0 in range(0, x.shape[1], block):
            blk = x[i, j0:j0 + block]
            amax = max(f32(np.abs(blk).max()), f32(1e-4))
            s = pow2_ceil(f32(np.float32(amax) * np.float32(1.0 / 448.0)))
            for j in range(block):
                v = f32(np.float32(blk[j]) / np.float32(s))
                v = min(max(v, -448.0), 448.0)
                out[i, j0 + j] = nearest_even(v, E4M3) * s
    return out


def fq_fp4_ue8m0(x, block=32):
    out = np.empty_like(x)
    for i in range(x.shape[0]):
        for j0 in range(0, x.shape[1], block):
            blk = x[i, j0:j0 + block]
            amax = max(f32(np.abs(blk).max()), f32(6.0 * 2.0 ** -126))
            s = pow2_ceil(f32(np.float32(amax) * np.float32(1.0 / 6.0)))
            for j in range(block):
                v = f32(np.float32(blk[j]) / np.float32(s))
                v = min(max(v, -6.0), 6.0)
                out[i, j0 + j] = nearest_even(v, E2M1) * s
    return out


def fq_fp4_e4m3(x, block=16):
    out = np.empty_like(x)
    for i in range(x.shape[0]):
        for j0 in range(0, x.shape[1], block):
            blk = x[i, j0:j0 + block]
            amax = max(f32(np.abs(blk).max()), f32(6.0 * 2.0 ** -9))
            s = nearest_even(f32(np.float32(amax) / np.float32(6.0)), E4M3)
            for j in range(block):
                v = f32(np.float32(blk[j]) / np.float32(s))
                v = min(max(v, -6.0), 6.0)
                out[i, j0 + j] = f32(nearest_even(v, E2M1) * s)
    return out


def main():
    xs = reference_inputs() + [fp4_tie_inputs()]
    arrays = {}
    for n, x in enumerate(xs):
        arrays[f"x{n}"] = x
        arrays[f"fp8_ue8m0_{n}"] = fq_fp8_ue8m0(x).astype(F32)
        arrays[f"fp4_ue8m0_{n}"] = fq_fp4_ue8m0(x).astype(F32)
        arrays[f"fp4_e4m3_{n}"] = fq_fp4_e4m3(x).astype(F32)
    path = os.path.join(HERE, "fakequant_kat.npz")
    np.savez_compressed(path, **arrays)
    print("wrote", path, {k: v.shape for k, v in arrays.items()})


if __name__ == "__main__":
    main()
