#!/usr/bin/env python3
"""Writes tests/golden/packer.npz: int8 weight-packing vectors whose expected
codes and scales come from exact rational arithmetic, not from any packer.

The packer being pinned is edgecore/ecm.py:50-59 (quantize_int8_symmetric):
per row, in float64, scale = max|w| / 127 (1.0 when that is 0); code =
clip(rint(w / scale), -128, 127) with rint rounding half to even; the scale is
stored as float32(scale).  Each float64 operation is one IEEE operation,
i.e. the exact result rounded to the nearest double, so the expected value of
every element is computed here as

    s64  = nearest double to Fraction(maxabs) / 127
    q64  = nearest double to Fraction(w) / Fraction(s64)
    code = round-half-even(q64), clipped

with Python's Fraction (exact) and float(Fraction) (correctly rounded).

Non-finite rows follow numpy: max() propagates NaN, so a row holding NaN has
scale NaN and every quotient NaN; an infinite maxabs gives scale inf, finite
elements quotient 0 and infinite ones inf/inf = NaN.  numpy's float64 ->
int32 cast of NaN gives INT32_MIN on x86-64 (cvttsd2si's "integer
indefinite"), which the clip maps to -128.

Rows:
  * adversarial: for random float32 maxabs values and codes k, elements whose
    quotient lies within a few ulps of k + 0.5, kept only where a plausible
    mistaken packer gives another code: float32 arithmetic throughout,
    division by the float32-rounded scale, or multiplication by 127 / maxabs;
  * exact .5 ties (maxabs 127 -> scale 1), +-maxabs -> +-127, a zero row;
  * seeded N(0, 0.02) rows (the generator's distribution);
  * NaN and infinity rows.
"""
from fractions import Fraction
from pathlib import Path

import numpy as np

COLS = 64
OUT = Path(__file__).resolve().parent / "packer.npz"


def exact_row(row: np.ndarray):
    """Expected (codes int8[COLS], scale float32) of one float32 row."""
    vals = [float(v) for v in row]
    if any(np.isnan(v) for v in vals):
        return np.full(len(vals), -128, np.int8), np.float32(np.nan)
    m = max(abs(v) for v in vals)
    if np.isinf(m):
        codes = [-128 if np.isinf(v) else 0 for v in vals]
        return np.array(codes, np.int8), np.float32(np.inf)
    s64 = float(Fraction(m) / 127) if m != 0 else 0.0
    if s64 == 0.0:
        s64 = 1.0
    codes = []
    for v in vals:
        q64 = float(Fraction(v) / Fraction(s64))
        c = round(q64)  # Python rounds an exact double half to even
        codes.append(min(127, max(-128, c)))
    return np.array(codes, np.int8), np.float32(s64)


# plausible mistakes (numpy, vectorised over a row)
def mistake_f32(row):
    r = row.astype(np.float32)
    m = np.max(np.abs(r))
    s = np.float32(m) / np.float32(127.0)
    s = np.float32(1.0) if s == 0 else s
    return np.clip(np.rint(r / s), -128, 127).astype(np.int8)


def mistake_f32_scale(row):
    a = row.astype(np.float64)
    s = np.max(np.abs(a)) / 127.0
    s = 1.0 if s == 0 else s
    return np.clip(np.rint(a / np.float64(np.float32(s))), -128, 127).astype(np.int8)


def mistake_reciprocal(row):
    a = row.astype(np.float64)
    m = np.max(np.abs(a))
    r = 127.0 / m if m != 0 else 1.0
    return np.clip(np.rint(a * r), -128, 127).astype(np.int8)


MISTAKES = (mistake_f32, mistake_f32_scale, mistake_reciprocal)


def adversarial_rows(rng, n_rows: int):
    rows = []
    found = {f.__name__: 0 for f in MISTAKES}
    while len(rows) < n_rows:
        m = np.float32(rng.uniform(1e-3, 0.2))
        s64 = float(Fraction(float(m)) / 127)
        elems = []
        tries = 0
        while len(elems) < COLS - 1 and tries < 4000:
            tries += 1
            k = int(rng.integers(-127, 127))
            base = np.float32((k + 0.5) * s64)
            cands = [base]
            lo = hi = base
            for _ in range(3):
                lo = np.nextafter(lo, np.float32(-np.inf))
                hi = np.nextafter(hi, np.float32(np.inf))
                cands += [lo, hi]
            for a in cands:
                if abs(float(a)) > float(m):
                    continue
                row = np.array([m, a], np.float32)
                want = exact_row(row)[0][1]
                bad = [f.__name__ for f in MISTAKES if f(row)[1] != want]
                if bad:
                    for b in bad:
                        found[b] += 1
                    elems.append(a)
                    break
        if len(elems) < COLS - 1:
            continue
        rows.append(np.array([m] + elems[: COLS - 1], np.float32))
    return rows, found


def main():
    rng = np.random.default_rng(20261202)
    rows, found = adversarial_rows(rng, 24)
    special = np.zeros((6, COLS), np.float32)
    special[0, :8] = [127, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, -127]  # scale exactly 1.0: ties to even
    special[1, :4] = [0.3, -0.7, 0.7, 0.05]                          # +-maxabs -> +-127
    # special[2] stays zero: scale 1, codes 0
    special[3, :4] = [0.1, np.nan, -0.2, 0.0]                         # NaN row
    special[4, :4] = [0.5, np.inf, -0.25, -np.inf]                    # infinite maxabs
    special[5, :4] = [-1e-40, 3e-41, 0.0, -7e-45]                     # subnormal maxabs
    seeded = rng.normal(0.0, 0.02, (64, COLS)).astype(np.float32)
    w = np.concatenate([np.stack(rows), special, seeded]).astype(np.float32)
    q = np.zeros(w.shape, np.int8)
    s = np.zeros(w.shape[0], np.float32)
    for i in range(w.shape[0]):
        q[i], s[i] = exact_row(w[i])
    np.savez_compressed(OUT, w=w, q=q, s=s, n_adversarial=len(rows))
    print(f"wrote {OUT}: {w.shape[0]} rows x {COLS}; adversarial rows {len(rows)}; "
          f"elements caught per mistaken packer: {found}")


if __name__ == "__main__":
    main()
