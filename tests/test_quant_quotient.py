"""The kernels' division-free fake-quant code (gs_device.h ``quant_code``)
against the IEEE division that the reference's fake-quant uses
(src/gru_qat/ste.py:65-95: ``torch.round(x / scale)``).

The steps are restated here in fp32 with an exact fma (rational arithmetic,
rounded once to fp32):

  q0 = clamp(fl(x * inv), -2^24, 2^24),  inv = fl(1 / s)
  r  = fma(-q0, s, x)
  q  = fma(r, inv, q0)

and ``clamp(rint(q), qmin, qmax) * s`` must equal
``clamp(rint(x / s), qmin, qmax) * s`` bit for bit. The inputs are chosen to
break a wrong restatement: values within a few ulps of every rounding
boundary (k + 1/2) s, exact multiples k s, random values over many binades,
zeros, subnormals, infinities and NaN, over scales at both ends of the
accepted range [2^-126, 2^64]. Dropping the correction step (q = q0) fails
on the near-boundary values, which the last test checks. The same kernel
function runs on the GPU in test_gpu_input_proj.py against torch's division.
"""

from __future__ import annotations

from fractions import Fraction

import numpy as np
import pytest

F32 = np.float32


def _rn32(v: Fraction) -> np.float32:
    """Round an exact rational to the nearest fp32, ties to even."""
    if v == 0:
        return F32(0.0)
    with np.errstate(over="ignore"):
        guess = F32(float(v))  # float(Fraction) is correctly rounded to fp64; fp64 -> fp32 may double-round
    if not np.isfinite(guess):
        return guess
    best = None
    for c in (np.nextafter(guess, F32(-np.inf)), guess, np.nextafter(guess, F32(np.inf))):
        if not np.isfinite(c):
            continue
        d = abs(Fraction(float(c)) - v)
        key = (d, int(np.frombuffer(c.tobytes(), np.uint32)[0]) & 1)  # ties: even mantissa
        if best is None or key < best[0]:
            best = (key, c)
    return best[1]


def _fma32(a: np.float32, b: np.float32, c: np.float32) -> np.float32:
    if not (np.isfinite(a) and np.isfinite(b) and np.isfinite(c)):
        with np.errstate(all="ignore"):
            return F32(np.float64(a) * np.float64(b) + np.float64(c))  # IEEE specials: no rounding involved
    return _rn32(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c)))


def _code_kernel(x: np.float32, s: np.float32, correct: bool = True) -> np.float32:
    inv = F32(F32(1.0) / s)
    with np.errstate(all="ignore"):
        q0 = F32(x * inv)
    q0 = F32(min(max(q0, F32(-2.0 ** 24)), F32(2.0 ** 24))) if not np.isnan(q0) else q0
    if not correct:
        return np.rint(q0)
    r = _fma32(F32(-q0), s, x)
    return np.rint(_fma32(r, inv, q0))


def _fq(code: np.float32, s: np.float32, lo: float, hi: float) -> np.float32:
    # fminf(fmaxf(v, lo), hi): NaN goes to lo, as with the reference kernel's
    # tl.minimum(tl.maximum(q, qmin), qmax) (scan.py:136-139)
    v = F32(lo) if np.isnan(code) else F32(min(max(code, F32(lo)), F32(hi)))
    return F32(v * s)


def _fq_ieee(x: np.float32, s: np.float32, lo: float, hi: float) -> np.float32:
    with np.errstate(all="ignore"):
        return _fq(np.rint(F32(x / s)), s, lo, hi)


SCALES = [F32(1.0 / 127.0), F32(1.0 / 255.0), F32(0.02), F32(3.0), F32(1e-8), F32(2.0 ** -126),
          F32(2.0 ** 64), np.nextafter(F32(1.0), F32(0.0)), np.nextafter(F32(1.0), F32(2.0)), F32(0.0123456)]
RANGES = [(-127, 127), (-128, 127), (-8, 7), (-4194304, 4194304)]


def _inputs(s: np.float32, rng: np.random.Generator) -> list:
    xs = []
    ks = np.concatenate([np.arange(-130, 131), rng.integers(-4194304, 4194304, 64)])
    for k in ks:
        for base in (F32((k + 0.5) * float(s)), F32(k * float(s))):
            v = base
            xs.append(v)
            up, dn = v, v
            for _ in range(3):
                up = np.nextafter(up, F32(np.inf))
                dn = np.nextafter(dn, F32(-np.inf))
                xs += [up, dn]
    with np.errstate(all="ignore"):
        xs += list(F32(rng.standard_normal(400) * float(s) * 10.0 ** rng.uniform(-3, 6, 400)))
    xs += [F32(0.0), F32(-0.0), F32(2.0 ** -149), F32(-(2.0 ** -149)), F32(np.inf), F32(-np.inf), F32(np.nan),
           F32(3.4e38), F32(-3.4e38)]
    return [x for x in xs]


@pytest.mark.parametrize("s", SCALES, ids=[f"s={float(s):.3g}" for s in SCALES])
def test_quotient_code_matches_ieee_division(s):
    rng = np.random.default_rng(int(np.frombuffer(s.tobytes(), np.uint32)[0]))
    xs = _inputs(s, rng)
    checked = 0
    for x in xs:
        code = _code_kernel(x, s)
        for lo, hi in RANGES:
            a, b = _fq(code, s, lo, hi), _fq_ieee(x, s, lo, hi)
            same = (a == b) or (np.isnan(a) and np.isnan(b))
            assert same, f"s={s!r} x={x!r} range=({lo},{hi}): kernel {a!r} != IEEE {b!r}"
            checked += 1
    assert checked > 4000


def test_uncorrected_product_is_not_enough():
    """fl(x * fl(1/s)) alone misrounds some near-boundary values; the
    correction step is what makes the codes exact."""
    misses = 0
    for s in SCALES[:5]:
        rng = np.random.default_rng(1)
        for x in _inputs(s, rng):
            if not np.isfinite(x):
                continue
            with np.errstate(all="ignore"):
                if np.rint(F32(x / s)) != _code_kernel(x, s, correct=False):
                    misses += 1
    assert misses > 0
