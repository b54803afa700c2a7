"""The compaction divides a row's pooled values by its normalizer n without a
division per value: with r = RN(1/n), q = RN(a*r), e = fma(-q, n, a) (exact) and
q' = fma(e, r, q), q' is the correctly rounded a/n (Markstein's theorem), which the
kernel uses for every value in [2^-100, FLT_MAX] and normalizers in [1, 2^16]
(csrc/segment.hip, divide_by_normalizer).  Checked here in exact rational arithmetic
with one rounding per operation, for integer counts and fractional masses in
[1, 2^16], random values, values next to exact quotients, sparse mantissas and the
ends of that range."""
import random
from fractions import Fraction

import numpy as np


def rn32(x: Fraction) -> np.float32:
    """Round-to-nearest-even of an exact rational to float32."""
    if x == 0:
        return np.float32(0.0)
    f = np.float32(float(x))
    best = None
    with np.errstate(over="ignore"):  # the neighbours of FLT_MAX include inf
        cands = (np.nextafter(f, np.float32(-np.inf)), f, np.nextafter(f, np.float32(np.inf)))
    for c in cands:
        if not np.isfinite(c):
            continue
        d = abs(Fraction(float(c)) - x)
        even = (int(np.float32(c).view(np.uint32)) & 1) == 0
        if best is None or d < best[0] or (d == best[0] and even):
            best = (d, c)
    return np.float32(best[1])


def corrected_quotient(a: np.float32, n: np.float32) -> np.float32:
    fa, fn = Fraction(float(a)), Fraction(float(n))
    r = rn32(1 / fn)
    q = rn32(fa * Fraction(float(r)))
    e = rn32(fa - Fraction(float(q)) * fn)                      # fma(-q, n, a)
    return rn32(Fraction(float(q)) + Fraction(float(e)) * Fraction(float(r)))  # fma(e, r, q)


def test_markstein_corrected_quotient_is_the_rounded_division():
    rng = random.Random(11)
    divisors = [np.float32(b) for b in (1, 2, 3, 5, 7, 9, 11, 13, 27, 31, 63, 1023, 65535, 65536)]
    divisors += [np.float32(1 + rng.random() * 20) for _ in range(8)]
    divisors += [np.float32(rng.uniform(1, 65536)) for _ in range(4)]
    checked = 0
    for n in divisors:
        fn = Fraction(float(n))
        values = [np.float32(rng.uniform(1, 2) * 2.0 ** rng.randint(-100, 127) * rng.choice((-1, 1)))
                  for _ in range(40)]
        values += [rn32(fn * Fraction(float(np.float32(rng.uniform(1, 2) * 2.0 ** rng.randint(-90, 100)))))
                   for _ in range(20)]
        values += [np.float32((rng.randint(1, 1 << 12) << rng.randint(0, 11)) * 2.0 ** rng.randint(-90, 90))
                   for _ in range(20)]
        values += [np.float32(2.0 ** -100), np.float32(-(2.0 ** -100) * 1.5), np.float32(3.4028234e38),
                   np.float32(-3.4028234e38)]
        for a in values:
            if not (2.0 ** -100 <= abs(float(a)) <= 3.4028234663852886e38):
                continue
            assert corrected_quotient(a, n) == rn32(Fraction(float(a)) / fn), (a, n)
            checked += 1
    assert checked > 1500
