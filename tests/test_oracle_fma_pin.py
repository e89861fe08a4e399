"""Pins the rounding sequence of the oracle's FMA-chain dot (orc_dot_fma).

The reference's restricted head scores a candidate as
``score = fmaf(hidden[f], embedding[f], score)`` for f = 0 .. H-1
(src/cuda/greedy.cu:171-176; its test oracle restates the same loop,
tests/cuda/cuda_tests.cu:739-744).  Each step is ONE rounding of the exact
value h*e + s to binary32, nearest-even.  This test evaluates that sequence in
exact rational arithmetic (fractions.Fraction, with a rounding function written
from the IEEE 754 definition) and requires the oracle to match it bit for bit
on rows whose values span many binades.

So that the check is known to be sensitive, the same inputs are evaluated in
the orders a plausible restatement mistake would produce -- the chain reversed,
the chain unfused (product rounded, then the sum), an 8-way strided chain
summed at the end, and a pairwise tree -- and each must differ from the
reference sequence on at least one row.
"""
from fractions import Fraction

import numpy as np

import oracle

H = 576
ROWS = 24


def rne32(v: Fraction) -> np.float32:
    """Exact value -> nearest binary32, ties to even (IEEE 754 roundTiesToEven),
    with subnormals and overflow to infinity."""
    if v == 0:
        return np.float32(0.0)
    sign = -1.0 if v < 0 else 1.0
    a = -v if v < 0 else v
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if a < Fraction(2) ** e:
        e -= 1
    elif a >= Fraction(2) ** (e + 1):
        e += 1
    e = max(e, -126)            # below the normal range the quantum stays 2^-149
    q = e - 23                  # quantum of binary32 in [2^e, 2^(e+1))
    m = a / Fraction(2) ** q
    n = m.numerator // m.denominator
    rem = m - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    if n * Fraction(2) ** q >= Fraction(2) ** 128:
        return np.float32(sign * np.inf)
    return np.float32(sign * float(n) * 2.0 ** q)   # exact: n < 2^25


def fma_chain(h, e, idx):
    s = np.float32(0.0)
    for f in idx:
        s = rne32(Fraction(float(h[f])) * Fraction(float(e[f])) + Fraction(float(s)))
    return s


def unfused_chain(h, e):
    s = np.float32(0.0)
    for f in range(h.size):
        p = rne32(Fraction(float(h[f])) * Fraction(float(e[f])))
        s = rne32(Fraction(float(s)) + Fraction(float(p)))
    return s


def strided8(h, e):
    parts = [fma_chain(h, e, range(j, h.size, 8)) for j in range(8)]
    s = np.float32(0.0)
    for p in parts:
        s = rne32(Fraction(float(s)) + Fraction(float(p)))
    return s


def pairwise(h, e):
    vals = [rne32(Fraction(float(h[f])) * Fraction(float(e[f]))) for f in range(h.size)]
    while len(vals) > 1:
        nxt = [rne32(Fraction(float(vals[i])) + Fraction(float(vals[i + 1])))
               for i in range(0, len(vals) - 1, 2)]
        if len(vals) % 2:
            nxt.append(vals[-1])
        vals = nxt
    return vals[0]


def rows():
    """Hidden rows in FP32 and FP16 embedding rows whose entries span many
    binades (scaled by 2^k per element), so partial sums cancel and round
    at every scale."""
    rng = np.random.default_rng(20260517)
    hs, es = [], []
    for _ in range(ROWS):
        h = (rng.standard_normal(H) * np.exp2(rng.integers(-8, 9, H))).astype(np.float32)
        e = (rng.standard_normal(H) * 0.02 * np.exp2(rng.integers(-6, 7, H)))
        e = np.clip(e, -60000, 60000).astype(np.float16)
        hs.append(h)
        es.append(e)
    return hs, es


def bits(v) -> int:
    return int(np.asarray(v, np.float32).view(np.uint32))


def test_rne32_against_numpy_double_to_float_on_doubles():
    """The rounding helper agrees with numpy's IEEE cast wherever the exact
    value is a double (numpy rounds double -> float32 correctly)."""
    rng = np.random.default_rng(3)
    vals = np.concatenate([rng.standard_normal(2000) * np.exp2(rng.integers(-140, 120, 2000)),
                           [2.0 ** -149 * 1.5, 2.0 ** -149 * 2.5, 3.4028235677973366e38,
                            3.4028235677973366e38 * (1 + 2 ** -25), 1.0 + 2 ** -24,
                            1.0 + 3 * 2 ** -24, -(1.0 + 2 ** -24)]])
    for v in vals:
        with np.errstate(over="ignore"):
            want = np.float32(v)
        assert bits(rne32(Fraction(float(v)))) == bits(want), v


def test_orc_dot_fma_is_the_ascending_single_rounding_chain():
    hs, es = rows()
    for h, e in zip(hs, es):
        want = fma_chain(h, e, range(H))
        got = oracle.dot(h, e.view(np.uint16), oracle.ORDER_FMA_CHAIN)
        assert bits(got) == bits(want)


def test_the_check_rejects_other_orders():
    """Each plausible wrong order differs from the reference sequence on at
    least one of the rows above, so the previous test would catch it."""
    hs, es = rows()
    want = [bits(fma_chain(h, e, range(H))) for h, e in zip(hs, es)]
    variants = {
        "reversed": [bits(fma_chain(h, e, range(H - 1, -1, -1))) for h, e in zip(hs, es)],
        "unfused": [bits(unfused_chain(h, e)) for h, e in zip(hs, es)],
        "strided8": [bits(strided8(h, e)) for h, e in zip(hs, es)],
        "pairwise": [bits(pairwise(h, e)) for h, e in zip(hs, es)],
    }
    for name, got in variants.items():
        assert got != want, f"{name} chain is indistinguishable on these inputs"


def test_orc_dot_mul_add_is_the_unfused_chain():
    """The mul-add order (operators.cpp:584-595) is also pinned by exact
    arithmetic here, beside its bit-exact check against oracle/_ref."""
    hs, es = rows()
    for h, e in list(zip(hs, es))[:6]:
        got = oracle.dot(h, e.view(np.uint16), oracle.ORDER_MUL_ADD_CHAIN)
        assert bits(got) == bits(unfused_chain(h, e))
