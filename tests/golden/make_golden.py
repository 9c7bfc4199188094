"""Write tests/golden/quant_golden.npz: small known-answer vectors for the quantized linear.

Expected values are computed with exact rational arithmetic (fractions.Fraction) and an
exact round-to-nearest-even into each floating type, i.e. independently of numpy's and
torch's float kernels. They pin the closed forms of LocalStrm's
src/kernels/quantization.py:
  dequant  (:104-122)  W = round_T( T(q) * round_T(scale[n, k // g]) )
  forward  (:129-141)  y = round_T( sum_k x_T[m,k] W[n,k] + round_T(bias[n]) )
The reference itself ships no tensor fixtures; inputs here are drawn from a seeded
numpy generator. Run: python tests/golden/make_golden.py
"""

from __future__ import annotations

import os
from fractions import Fraction

import numpy as np

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "quant_golden.npz")

# (fraction bits, minimum normal exponent) per type
FMT = {"f32": (23, -126), "f16": (10, -14), "bf16": (7, -126)}


def round_exact(v: Fraction, fmt: str) -> Fraction:
    """Exact IEEE round-to-nearest-even of a rational into `fmt` (no overflow handling;
    the vectors stay far from the largest finite values)."""
    mant, emin = FMT[fmt]
    if v == 0:
        return Fraction(0)
    sign = -1 if v < 0 else 1
    a = abs(v)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    e = max(e, emin)
    quantum = Fraction(2) ** (e - mant)
    t = a / quantum
    n = t.numerator // t.denominator
    rem = t - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    return sign * n * quantum


def fr(x) -> Fraction:
    return Fraction(float(x))


def to_f32_array(vals) -> np.ndarray:
    return np.array([float(v) for v in vals], dtype=np.float64).astype(np.float32)


def case(rng, name, n, k, kind, group, scale_fmt):
    if kind == "int8":
        q = rng.integers(-128, 128, size=(n, k), dtype=np.int64)
    else:
        q = rng.integers(-8, 8, size=(n, k), dtype=np.int64)
    g = 1 if group is None else -(-k // group)
    scale = rng.uniform(0.001, 0.05, size=(n, g)).astype(np.float32)
    if scale_fmt == "bf16":
        scale = np.array([[float(round_exact(fr(s), "bf16")) for s in row] for row in scale],
                         dtype=np.float32)
    x = rng.standard_normal(size=(3, k)).astype(np.float32)
    bias = rng.standard_normal(size=(n,)).astype(np.float32) * np.float32(0.1)
    rec = {
        f"{name}/q": q.astype(np.int8),
        f"{name}/scale": scale,
        f"{name}/x": x,
        f"{name}/bias": bias,
        f"{name}/meta": np.array([n, k, -1 if group is None else group], dtype=np.int64),
    }
    for t in ("f32", "f16", "bf16"):
        w = []
        for i in range(n):
            row = []
            for j in range(k):
                s = scale[i, 0 if group is None else j // group]
                s_t = round_exact(fr(s), t)
                row.append(round_exact(Fraction(int(q[i, j])) * s_t, t))
            w.append(row)
        rec[f"{name}/w_{t}"] = np.array([[float(v) for v in row] for row in w], dtype=np.float32)
        xs = [[round_exact(fr(v), t) for v in row] for row in x]
        b_t = [round_exact(fr(b), t) for b in bias]
        y_exact = []
        for mi in range(x.shape[0]):
            y_exact.append([sum((xs[mi][j] * w[i][j] for j in range(k)), Fraction(0)) + b_t[i]
                            for i in range(n)])
        rec[f"{name}/y_{t}_exact"] = np.array([[float(v) for v in row] for row in y_exact])
        rec[f"{name}/y_{t}"] = np.array([[float(round_exact(v, t)) for v in row] for row in y_exact],
                                        dtype=np.float32)
        rec[f"{name}/x_{t}"] = np.array([[float(v) for v in row] for row in xs], dtype=np.float32)
    return rec


def main() -> None:
    rng = np.random.default_rng(20240601)
    recs = {}
    recs.update(case(rng, "int8_pc", 16, 32, "int8", None, "f32"))
    recs.update(case(rng, "int4_pc_oddk", 16, 33, "int4", None, "f32"))
    recs.update(case(rng, "int4_g16", 16, 64, "int4", 16, "bf16"))
    recs.update(case(rng, "int4_g128", 32, 256, "int4", 128, "bf16"))
    recs.update(case(rng, "int8_k256", 32, 256, "int8", None, "f32"))
    recs.update(case(rng, "int4_pc_k128", 24, 128, "int4", None, "f32"))
    np.savez_compressed(OUT, **recs)
    print(OUT, len(recs), "arrays")


if __name__ == "__main__":
    main()
