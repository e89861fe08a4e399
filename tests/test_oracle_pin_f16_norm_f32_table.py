"""Independent pins for two oracle pieces that the other oracle tests reach
only through the oracle itself:

* ``orc_rms_norm_f16`` (oracle.c).  This build defines the FP16 RMSNorm as
  "the FP32 CPU order (src/cpu/operators.cpp:523-535) on the decoded inputs,
  output rounded to nearest-even half".  Checked here against exactly that
  definition built from two independent parts: the reference's own
  ``rms_norm_f32`` compiled from its sources (oracle/_ref) and numpy's IEEE
  float32 -> float16 cast.  The rows include outputs in the half subnormal
  range and outputs that overflow to infinity.
* The FP32-table branch of the oracle's dot (``dot_in_order_f32``, the cfg1
  path: src/cpu/smollm2.cpp:437-439 materializes FP32 weights), reached
  through ``oracle.decode_tail`` with a float32 table and one candidate per
  row, so the reported score is the candidate's chain.  Both orders are
  evaluated in exact rational arithmetic (the reference CUDA head's
  ``fmaf`` chain, src/cuda/greedy.cu:171-176, and ``linear_f32``'s unfused
  chain, src/cpu/operators.cpp:584-595) and must match bit for bit; the
  reversed, unfused, strided and pairwise variants must each differ from the
  FMA chain on these rows, so the check is known to be sensitive.
"""
import numpy as np
import pytest

import oracle
from tests import cases
from tests.test_oracle_fma_pin import (bits, fma_chain, pairwise, strided8,
                                       unfused_chain)


def _ref():
    r = oracle.ref()
    if r is None:
        pytest.skip("oracle/_ref not built (reference tree absent when built)")
    return r


def _ref_norm_f32(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    rows, hidden = x.shape
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    y = np.empty_like(x)
    assert _ref().mfref_rms_norm_f32(x.ctypes.data, w.ctypes.data, eps, y.ctypes.data,
                                     rows, hidden) == 0
    return y


def _big_case():
    """64 rows of 576: enough elements that orders one FP32 ulp apart round
    to different halves somewhere."""
    rng = np.random.default_rng(99)
    x = rng.standard_normal((64, 576)).astype(np.float16)
    w = (1.0 + 0.02 * rng.standard_normal(576)).astype(np.float16)
    return x.view(np.uint16), w.view(np.uint16)


def _half_cases():
    """(x16 bits, w16 bits) pairs: the reference test shapes with N(0,1)
    inputs and 1 + N(0, 0.02) weights, a larger block, plus rows built to
    land outputs in the half subnormal range and past the half range."""
    rng = np.random.default_rng(1234)
    out = [_big_case()]
    for rows, hidden in cases.RMS_SHAPES:
        x = rng.standard_normal((rows, hidden)).astype(np.float16)
        w = (1.0 + 0.02 * rng.standard_normal(hidden)).astype(np.float16)
        out.append((x.view(np.uint16), w.view(np.uint16)))
    hidden = 576
    x = rng.standard_normal((4, hidden)).astype(np.float16)
    # weights spanning half subnormals (2^-24 .. 2^-15) up to 2^14, so the
    # products (x * inv) * w fall below the normal range and near the top
    w = (rng.choice([-1.0, 1.0], hidden) *
         np.exp2(rng.integers(-26, 15, hidden)) *
         (1.0 + rng.random(hidden))).astype(np.float16)
    out.append((x.view(np.uint16), w.view(np.uint16)))
    # one dominant feature: x * inv ~ sqrt(H) = 24, times w = 60000 overflows
    x = np.full((2, hidden), 1e-3, np.float16)
    x[:, 7] = 3.0
    x[1, 7] = -3.0
    w = np.full(hidden, 60000.0, np.float16)
    out.append((x.view(np.uint16), w.view(np.uint16)))
    return out


def test_rms_norm_f16_is_rne_half_of_the_reference_f32_norm():
    eps = 1e-5
    saw_sub = saw_inf = False
    for x16, w16 in _half_cases():
        got = oracle.rms_norm_f16(x16, w16, eps)
        x32 = x16.view(np.float16).astype(np.float32)
        w32 = w16.view(np.float16).astype(np.float32)
        y32 = _ref_norm_f32(x32, w32, eps)
        with np.errstate(over="ignore"):
            want = y32.astype(np.float16).view(np.uint16)
        assert np.array_equal(got, want)
        mag = got & 0x7FFF
        saw_sub |= bool(np.any((mag > 0) & (mag < 0x0400)))
        saw_inf |= bool(np.any(mag == 0x7C00))
    assert saw_sub and saw_inf, "the edge rows must reach subnormal and overflowed halves"


def test_rms_norm_f16_output_is_the_nearest_half_to_the_reference_f32_norm():
    """The reference's GPU test bounds its FP32 norm by 3e-5 against the CPU
    loop (tests/cuda/cuda_tests.cu:140); a half output cannot meet an
    absolute 3e-5 (the half quantum at 1.0 is 2^-10), so the FP16 op is held
    to the tightest bound there is: no half lies closer to the FP32 CPU
    norm than the oracle's output, and the FP32 values behind it are the
    CPU loop's own (within 3e-5, in fact equal)."""
    eps = 1e-5
    x16, w16 = _big_case()
    got = oracle.rms_norm_f16(x16, w16, eps).view(np.float16).astype(np.float64)
    x32 = x16.view(np.float16).astype(np.float32)
    w32 = w16.view(np.float16).astype(np.float32)
    y32 = _ref_norm_f32(x32, w32, eps)
    assert np.max(np.abs(oracle.rms_norm_f32(x32, w32, eps) - y32)) <= 3e-5
    ref = y32.astype(np.float64)
    err = np.abs(got - ref)
    up = np.nextafter(got.astype(np.float16), np.float16(np.inf)).astype(np.float64)
    dn = np.nextafter(got.astype(np.float16), np.float16(-np.inf)).astype(np.float64)
    assert np.all(err <= np.abs(up - ref)) and np.all(err <= np.abs(dn - ref))


def test_rms_norm_f16_check_rejects_other_orders():
    """x * (inv * w) and a sum of squares in another order must differ from
    the reference on these rows, so the bit-exact check above would catch
    such a restatement."""
    eps = np.float32(1e-5)
    x16, w16 = _big_case()
    x = x16.view(np.float16).astype(np.float32)
    w = w16.view(np.float16).astype(np.float32)
    want = oracle.rms_norm_f16(x16, w16, float(eps))
    hidden = x.shape[1]

    def inv_of(sumsq):
        return np.float32(1.0) / np.sqrt(np.float32(sumsq) / np.float32(hidden) + eps)

    def seq_sum(v):
        s = np.float32(0.0)
        for t in v:
            s = np.float32(s + np.float32(t * t))
        return s

    reassoc = np.empty_like(want)
    pairsum = np.empty_like(want)
    for r in range(x.shape[0]):
        inv = np.float32(inv_of(seq_sum(x[r])))
        reassoc[r] = (x[r] * (inv * w)).astype(np.float16).view(np.uint16)
        inv2 = np.float32(inv_of(np.sum(x[r] * x[r], dtype=np.float32)))   # pairwise
        pairsum[r] = ((x[r] * inv2) * w).astype(np.float16).view(np.uint16)
    assert not np.array_equal(reassoc, want)
    assert not np.array_equal(pairsum, want)


def _f32_rows(rows=16, hidden=576):
    """Hidden rows and FP32 table rows whose entries span many binades."""
    rng = np.random.default_rng(20260602)
    hs = (rng.standard_normal((rows, hidden)) *
          np.exp2(rng.integers(-8, 9, (rows, hidden)))).astype(np.float32)
    es = (rng.standard_normal((rows, hidden)) * 0.02 *
          np.exp2(rng.integers(-10, 11, (rows, hidden)))).astype(np.float32)
    return hs, es


def _scores_via_decode_tail(hs, es, order):
    """One row per table row, each row's state allowing exactly its own token:
    the decode tail's score is then that token's chain over the FP32 table."""
    rows, hidden = hs.shape
    offsets = np.arange(rows + 1, dtype=np.uint32)
    tokens = np.arange(rows, dtype=np.uint32)
    states = np.arange(rows, dtype=np.uint32)
    tok, sc, _ = oracle.decode_tail(hs, None, 1e-5, es, states, offsets, tokens,
                                    order=order)
    assert np.array_equal(tok, tokens)
    return sc


@pytest.mark.parametrize("order", [oracle.ORDER_FMA_CHAIN, oracle.ORDER_MUL_ADD_CHAIN])
def test_f32_table_dot_is_the_reference_chain(order):
    hs, es = _f32_rows()
    got = _scores_via_decode_tail(hs, es, order)
    for r in range(hs.shape[0]):
        want = fma_chain(hs[r], es[r], range(hs.shape[1])) \
            if order == oracle.ORDER_FMA_CHAIN else unfused_chain(hs[r], es[r])
        assert bits(got[r]) == bits(want), (order, r)


def test_f32_table_check_rejects_other_orders():
    hs, es = _f32_rows()
    want = [bits(fma_chain(h, e, range(h.size))) for h, e in zip(hs, es)]
    variants = {
        "reversed": [bits(fma_chain(h, e, range(h.size - 1, -1, -1))) for h, e in zip(hs, es)],
        "unfused": [bits(unfused_chain(h, e)) for h, e in zip(hs, es)],
        "strided8": [bits(strided8(h, e)) for h, e in zip(hs, es)],
        "pairwise": [bits(pairwise(h, e)) for h, e in zip(hs, es)],
    }
    for name, got in variants.items():
        assert got != want, f"{name} chain is indistinguishable on these rows"
