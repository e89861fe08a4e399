"""Pins the CPU oracle (oracle/oracle.c) before anything is checked against it.

Each check is independent of the oracle's own formulas: the reference's own
test vectors and fixtures, the reference's CPU code compiled in place
(oracle/_ref), exact rational arithmetic, numpy's IEEE float16 casts and
float64 brute force.  A plausible restatement mistake (a transposed operand,
fused instead of unfused arithmetic, a wrong tie rule) fails at least one.
"""
import ctypes
import math
from fractions import Fraction

import numpy as np
import pytest

import oracle
from tests import cases
from market_sim_amd import workloads

INVALID = cases.INVALID


def needs_ref():
    r = oracle.ref()
    if r is None:
        pytest.skip("oracle/_ref (reference CPU build) not available")
    return r


# ------------------------------------------------------------ float16 ------

def test_half_to_float_exhaustive_matches_numpy():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ours = oracle.half_to_float(bits)
    theirs = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(theirs)
    assert np.array_equal(np.isnan(ours), nan)
    assert np.array_equal(ours[~nan].view(np.uint32), theirs[~nan].view(np.uint32))


def test_float_to_half_matches_numpy_rne():
    rng = np.random.default_rng(1)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(
            10.0) ** rng.integers(-9, 6, 20000).astype(np.float32),
        # halfway points between adjacent halves (ties to even) and neighbours
        (np.arange(0, 65504, 7.5, dtype=np.float32)),
        np.array([65504, 65519.99, 65520, 1e6, 5.96e-8, 2.98e-8, 2.9802322e-8,
                  2.9802326e-8, 8.94e-8, 6.1e-5, 6.097e-5, 0.0, -0.0, np.inf,
                  -np.inf], np.float32)])
    mids = (bits := np.arange(0x0000, 0x7bff, 3, dtype=np.uint16).view(np.float16)
            .astype(np.float32))
    nxt = (np.arange(0x0001, 0x7c00, 3, dtype=np.uint16).view(np.float16)
           .astype(np.float32))
    halfway = ((mids.astype(np.float64) + nxt.astype(np.float64)) / 2).astype(np.float32)
    vals = np.concatenate([vals, halfway, -halfway])
    ours = oracle.float_to_half_bits(vals)
    with np.errstate(over="ignore"):
        theirs = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(ours, theirs)


# ------------------------------------------------------------ RMSNorm ------

@pytest.mark.parametrize("rows,hidden", cases.RMS_SHAPES)
def test_rms_norm_bit_exact_vs_reference_cpu(rows, hidden):
    r = needs_ref()
    x, w = cases.rms_norm_case(rows, hidden)
    ours = oracle.rms_norm_f32(x, w, 1e-5)
    theirs = np.empty_like(x)
    assert r.mfref_rms_norm_f32(x.ctypes.data, w.ctypes.data, 1e-5,
                                theirs.ctypes.data, rows, hidden) == 0
    assert np.array_equal(ours.view(np.uint32), theirs.view(np.uint32))


def test_rms_norm_bit_exact_vs_reference_cpu_random():
    r = needs_ref()
    rng = np.random.default_rng(7)
    for hidden in (576, 2048, 1000):
        x = rng.standard_normal((5, hidden)).astype(np.float32) * np.float32(3)
        w = (1 + 0.02 * rng.standard_normal(hidden)).astype(np.float32)
        ours = oracle.rms_norm_f32(x, w, 1e-5)
        theirs = np.empty_like(x)
        assert r.mfref_rms_norm_f32(x.ctypes.data, w.ctypes.data, 1e-5,
                                    theirs.ctypes.data, 5, hidden) == 0
        assert np.array_equal(ours.view(np.uint32), theirs.view(np.uint32))


def test_rms_norm_hand_values():
    """tests/unit/cpu_operator_tests.cpp:59-84."""
    x = np.array([[1, 2, 3, 4], [-1, 0.5, 2, -3]], np.float32)
    w = np.array([1, 0.5, 2, 1.5], np.float32)
    y = oracle.rms_norm_f32(x, w, 1e-5)
    for row in range(2):
        sq = sum(float(v) ** 2 for v in x[row])  # exact for these values
        inv = 1.0 / math.sqrt(sq / 4.0 + 1e-5)
        for c in range(4):
            assert abs(float(y[row, c]) - float(x[row, c]) * inv * float(w[c])) < 1e-6


def test_rms_norm_sum_is_unfused_sequential():
    """A fused or reordered sum of squares changes the bits here: the chosen
    values make x*x inexact so every rounding step is visible."""
    r = needs_ref()
    rng = np.random.default_rng(3)
    x = (rng.random((1, 577)) * 1.37 + 0.11).astype(np.float32)
    w = np.ones(577, np.float32)
    ours = oracle.rms_norm_f32(x, w, 1e-5)
    theirs = np.empty_like(x)
    r.mfref_rms_norm_f32(x.ctypes.data, w.ctypes.data, 1e-5, theirs.ctypes.data, 1, 577)
    assert np.array_equal(ours, theirs)
    # the float64 value of the same formula differs in low bits, proving the
    # comparison above is sensitive to the accumulation precision
    s64 = float(np.sum(x.astype(np.float64) ** 2))
    inv64 = 1.0 / math.sqrt(s64 / 577 + 1e-5)
    y64 = (x.astype(np.float64) * inv64).astype(np.float32)
    assert not np.array_equal(y64, ours)


# ------------------------------------------------------------ linear -------

def test_linear_known_answer():
    """tests/unit/cpu_operator_tests.cpp:86-107: [1,2,3] x [[1,0,-1],[.5,.5,.5]]."""
    x = np.array([1, 2, 3], np.float32)
    w = cases.f16_bits(np.array([[1, 0, -1], [0.5, 0.5, 0.5]], np.float32))
    for order in (oracle.ORDER_FMA_CHAIN, oracle.ORDER_MUL_ADD_CHAIN):
        got = [float(oracle.dot(x, w[i], order)) for i in range(2)]
        assert got == [-2.0, 3.0]


def test_mul_add_order_bit_exact_vs_reference_linear_f32():
    r = needs_ref()
    rng = np.random.default_rng(11)
    rows, inf, outf = 3, 576, 257
    x = rng.standard_normal((rows, inf)).astype(np.float32)
    wb = (rng.standard_normal((outf, inf)) * 0.02).astype(np.float16).view(np.uint16)
    w32 = wb.view(np.float16).astype(np.float32)
    theirs = np.empty((rows, outf), np.float32)
    assert r.mfref_linear_f32(x.ctypes.data, np.ascontiguousarray(w32).ctypes.data,
                              theirs.ctypes.data, rows, inf, outf) == 0
    ours = np.array([[oracle.dot(x[i], wb[o], oracle.ORDER_MUL_ADD_CHAIN)
                      for o in range(outf)] for i in range(rows)], np.float32)
    assert np.array_equal(ours.view(np.uint32), theirs.view(np.uint32))
    # the fused order is a different function of the same inputs
    fused = np.array([[oracle.dot(x[i], wb[o], oracle.ORDER_FMA_CHAIN)
                       for o in range(outf)] for i in range(rows)], np.float32)
    assert not np.array_equal(fused, theirs)


def test_linear_f16_rounds_fp32_sum_to_half():
    x, w = cases.linear_case(3, 576, 64)
    out16, out32 = oracle.linear_f16(x, w)
    assert np.array_equal(out16, out32.astype(np.float16).view(np.uint16))
    exact = (x.view(np.float16).astype(np.float64) @
             w.view(np.float16).astype(np.float64).T)
    assert np.max(np.abs(out32 - exact)) < 1e-5


# ------------------------------------------------------ selection rules ----

def test_tiny_head_known_answer_exact_rationals():
    """tests/cuda/cuda_tests.cu:699-800: tokens [14, 8, 1]; scores checked
    against exact rational arithmetic (every product and partial sum is a
    multiple of 1/128 with small numerator, so any order is exact)."""
    c = cases.tiny_head_case()
    tok, sc = oracle.restricted_output_head_f16(c["hidden"], c["embedding"],
                                                c["allowed"], c["counts"],
                                                c["max_allowed"])
    assert tok.tolist() == [14, 8, 1]
    h = c["hidden"].view(np.float16).astype(np.float64)
    e = c["embedding"].view(np.float16).astype(np.float64)

    def exact(row, tkn):
        return sum(Fraction(h[row, f]) * Fraction(e[tkn, f]) for f in range(8))

    assert exact(0, 9) == Fraction(-0.2421875)
    assert exact(0, 3) == Fraction(-0.359375)
    assert exact(0, 14) == Fraction(0.375)
    assert exact(1, 6) == exact(1, 4) == Fraction(-0.109375)
    assert exact(1, 8) == Fraction(0.28125)
    assert float(sc[0]) == 0.375 and float(sc[1]) == 0.28125
    assert math.isnan(float(sc[2]))
    for order in (oracle.ORDER_FMA_CHAIN, oracle.ORDER_MUL_ADD_CHAIN):
        got = oracle.scores(h[0].astype(np.float32), c["embedding"],
                            np.array([9, 3, 14], np.uint32), order)
        assert got.tolist() == [-0.2421875, -0.359375, 0.375]


@pytest.mark.parametrize("rows,vocab", [(1, 17), (3, 49152)])
def test_greedy_f16_reference_cases(rows, vocab):
    """tests/cuda/cuda_tests.cu:508-565 and :1132-1135."""
    logits, expected = cases.greedy_case(rows, vocab)
    assert oracle.greedy_f16(logits).tolist() == expected.tolist()


def test_greedy_all_nan_row_writes_zero():
    """src/cuda/greedy.cu:57: a row with no comparable value selects 0."""
    logits = cases.f16_bits(np.full((1, 9), np.nan, np.float32))
    assert oracle.greedy_f16(logits).tolist() == [0]


def test_restricted_greedy_market_dfa_case():
    """tests/cuda/cuda_tests.cu:567-697 with the reference's market DFA."""
    c = cases.market_restricted_greedy_case()
    got = oracle.restricted_greedy_f16(c["logits"], c["allowed"], c["counts"],
                                       c["max_allowed"])
    vals = c["logits"].view(np.float16).astype(np.float32)
    for r, cands in enumerate(c["lists"]):
        if r <= 1:
            assert got[r] == cands.min()  # all equal / all NaN -> lowest id
        else:
            v = vals[r, cands]
            best = v.max()
            assert got[r] == cands[v == best].min()
        assert got[r] in set(cands.tolist())  # the 100.0 decoy is never chosen


def test_restricted_greedy_invalid_rows():
    """tests/cuda/cuda_tests.cu:1173-1255."""
    variants, vocab, max_allowed = cases.invalid_rows_greedy_case()
    for logits, allowed, counts in variants:
        got = oracle.restricted_greedy_f16(logits, allowed, counts, max_allowed)
        assert got.tolist() == [INVALID]


def test_restricted_head_invalid_rows():
    """tests/cuda/cuda_tests.cu:1341-1403."""
    c = cases.invalid_rows_head_case()
    tok, _ = oracle.restricted_output_head_f16(c["hidden"], c["embedding"],
                                               c["allowed"], c["counts"],
                                               c["max_allowed"])
    assert tok.tolist() == [INVALID] * 3


def test_real_smollm2_logits_fixture():
    """tests/fixtures/golden/smollm2-pr4-greedy-f32.*: FP32 logits of the
    real model -> [198, 198, 504] with the recorded top-2 margins; the legal
    sets of src/tools/cuda_smollm2_conformance.cu:85-107 give the same."""
    logits, tokens, margins = cases.real_logits()
    assert oracle.greedy_f32(logits).tolist() == tokens.tolist() == [198, 198, 504]
    srt = np.sort(logits, axis=1)
    assert np.allclose(srt[:, -1] - srt[:, -2], margins, rtol=0, atol=1e-6)
    allowed = np.array(cases.REAL_LEGAL_SETS, np.uint32)
    counts = np.full(3, 4, np.uint32)
    got = oracle.restricted_greedy_f32(logits, allowed, counts, 4)
    assert got.tolist() == [198, 198, 504]
    half = logits.astype(np.float16).view(np.uint16)
    assert oracle.greedy_f16(half).tolist() == [198, 198, 504]


def test_selection_nan_negzero_and_ties():
    """Rules of src/cuda/greedy.cu:96-100: -0 == +0 ties to the lower id; NaN
    never wins; -inf is a valid score."""
    v = np.array([[0.0, -0.0, np.nan, -np.inf]], np.float32)
    allowed = np.array([[3, 1, 0, 2]], np.uint32)
    counts = np.array([4], np.uint32)
    logits = np.full((1, 4), np.nan, np.float32)
    logits[0, allowed[0]] = v[0]
    assert oracle.restricted_greedy_f32(logits, allowed, counts, 4).tolist() == [1]
    logits[0, :] = [np.nan, np.nan, -np.inf, np.nan]
    assert oracle.restricted_greedy_f32(logits, allowed, counts, 4).tolist() == [2]
    logits[0, :] = np.nan
    assert oracle.restricted_greedy_f32(logits, allowed, counts, 4).tolist() == [0]


# ------------------------------------------------------------ DFA ----------

def _flatten(language):
    ids = np.array([c[0] for c in language], np.uint32)
    offs = np.zeros(len(language) + 1, np.uint32)
    toks = []
    for i, c in enumerate(language):
        toks.extend(c[1])
        offs[i + 1] = offs[i] + len(c[1])
    return ids, offs, np.array(toks or [0], np.uint32)


def test_token_dfa_known_answer_via_reference():
    """tests/unit/token_dfa_tests.cpp:22-49: 3 choices -> 7 states, 6 arcs,
    root allowed [3, 9], 9 -> 6 reaches choice 99."""
    r = needs_ref()
    ids, offs, toks = _flatten([(41, [9, 4]), (7, [3, 8, 1]), (99, [9, 6])])
    cap = 64
    o = np.zeros(cap, np.uint32); t = np.zeros(cap, np.uint32)
    n = np.zeros(cap, np.uint32); term = np.zeros(cap, np.uint32)
    ns, na = ctypes.c_uint32(), ctypes.c_uint32()
    rc = r.mfref_token_dfa_export(ids.ctypes.data, offs.ctypes.data, toks.ctypes.data,
                                  3, 64, 8, 16, 32, 32, o.ctypes.data, t.ctypes.data,
                                  n.ctypes.data, term.ctypes.data, cap, cap,
                                  ctypes.byref(ns), ctypes.byref(na))
    assert rc == 0 and ns.value == 7 and na.value == 6
    assert t[o[0]:o[1]].tolist() == [3, 9]
    # advance by the arc position, the way the device advance does it
    s = 0
    for token in (9, 6):
        row = t[o[s]:o[s + 1]].tolist()
        s = int(n[o[s] + row.index(token)])
    assert term[s] == 99


def test_market_dfa_fixture_properties():
    """tests/property/action_dfa_properties.cpp:24-104: 3230 states, 3229
    arcs, arcs strictly ascending, terminal <=> no arcs, max out-degree 11."""
    offsets, tokens, nxt = cases.market_dfa()
    assert offsets.size - 1 == 3230 and tokens.size == 3229
    deg = np.diff(offsets.astype(np.int64))
    assert deg.max() == 11 and (deg == 0).sum() == 1585
    for s in range(3230):
        row = tokens[offsets[s]:offsets[s + 1]]
        assert np.all(np.diff(row.astype(np.int64)) > 0)
    assert tokens[offsets[0]:offsets[1]].tolist() == [67, 5775, 27136]


def test_market_dfa_fixture_matches_reference_build():
    r = needs_ref()
    offsets, tokens, nxt = cases.market_dfa()
    cap = 8192
    o = np.zeros(cap, np.uint32); t = np.zeros(cap, np.uint32); n = np.zeros(cap, np.uint32)
    term = np.zeros(cap, np.uint32)
    ns, na = ctypes.c_uint32(), ctypes.c_uint32()
    assert r.mfref_market_dfa_export(o.ctypes.data, t.ctypes.data, n.ctypes.data,
                                     term.ctypes.data, cap, cap, ctypes.byref(ns),
                                     ctypes.byref(na)) == 0
    assert np.array_equal(o[:ns.value + 1], offsets)
    assert np.array_equal(t[:na.value], tokens) and np.array_equal(n[:na.value], nxt)
    assert np.array_equal(term[:ns.value], cases.market_dfa_terminal())
    lo = np.zeros(4096, np.uint32); lt = np.zeros(65536, np.uint32)
    ne, nt = ctypes.c_uint32(), ctypes.c_uint32()
    assert r.mfref_market_language(lo.ctypes.data, lt.ctypes.data, 4096, 65536,
                                   ctypes.byref(ne), ctypes.byref(nt)) == 0
    lang = [lt[lo[i]:lo[i + 1]].tolist() for i in range(ne.value)]
    assert lang == cases.market_language()


# -------------------------------------------------------- decode tail ------

def _margin_qualified_brute_force(w: workloads.Workload, y: np.ndarray):
    """float64 scores; returns (winner, top-2 margin, error bound) per row."""
    e64 = w.embedding.view(np.float16).astype(np.float64)
    out = []
    for r in range(w.rows):
        s = int(w.row_state[r])
        if s == workloads.STATE_UNRESTRICTED:
            ids = np.arange(w.vocab)
        else:
            ids = w.state_tokens[w.state_offsets[s]:w.state_offsets[s + 1]]
        sc = e64[ids] @ y[r].astype(np.float64)
        absd = np.abs(e64[ids]) @ np.abs(y[r].astype(np.float64))
        o = np.argsort(-sc, kind="stable")
        win = ids[o[0]]
        margin = sc[o[0]] - sc[o[1]] if ids.size > 1 else np.inf
        bound = 2 * (w.hidden * 2.0 ** -24) * absd.max() * 1.01
        out.append((int(win), margin, bound, float(sc[o[0]])))
    return out


@pytest.mark.parametrize("order", [oracle.ORDER_FMA_CHAIN, oracle.ORDER_MUL_ADD_CHAIN])
def test_decode_tail_vs_float64_brute_force(order):
    w = workloads.config(3, seed=5, scale_vocab=6000, scale_rows=40)
    tok, sc, nx = oracle.decode_tail(w.x, w.norm_weight, w.epsilon, w.embedding,
                                     w.row_state, w.state_offsets, w.state_tokens,
                                     order=order, threads=4)
    y = oracle.rms_norm_f32(w.x, w.norm_weight, w.epsilon)
    checked = 0
    for r, (win, margin, bound, s64) in enumerate(_margin_qualified_brute_force(w, y)):
        assert abs(float(sc[r]) - s64) <= bound
        if margin > bound:
            assert tok[r] == win
            checked += 1
    assert checked >= w.rows - 1


def test_decode_tail_one_hot_closed_form():
    """A one-hot normalized hidden makes each score one embedding column,
    exactly, in either order."""
    w = workloads.config(2, seed=2, scale_vocab=3000, scale_rows=8)
    x = np.zeros((w.rows, w.hidden), np.float32)
    cols = np.arange(w.rows) * 37 % w.hidden
    x[np.arange(w.rows), cols] = 1.0
    e32 = w.embedding.view(np.float16).astype(np.float32)
    for order in (oracle.ORDER_FMA_CHAIN, oracle.ORDER_MUL_ADD_CHAIN):
        tok, sc, _ = oracle.decode_tail(x, None, 1e-5, w.embedding, w.row_state,
                                        w.state_offsets, w.state_tokens, order=order)
        for r in range(w.rows):
            ids = w.state_tokens[w.state_offsets[r]:w.state_offsets[r + 1]]
            col = e32[ids, cols[r]]
            assert sc[r] == col.max()
            assert tok[r] == ids[col == col.max()].min()


def test_decode_tail_unrestricted_equals_all_ids_list():
    w = workloads.config(3, seed=9, scale_vocab=2000, scale_rows=12)
    assert (w.row_state == workloads.STATE_UNRESTRICTED).any()
    tok, sc, nx = oracle.decode_tail(w.x, w.norm_weight, w.epsilon, w.embedding,
                                     w.row_state, w.state_offsets, w.state_tokens)
    rs = np.zeros(w.rows, np.uint32)
    tok2, sc2, _ = oracle.decode_tail(w.x, w.norm_weight, w.epsilon, w.embedding,
                                      rs, np.array([0, w.vocab], np.uint32),
                                      np.arange(w.vocab, dtype=np.uint32))
    unr = w.row_state == workloads.STATE_UNRESTRICTED
    assert np.array_equal(tok[unr], tok2[unr])
    assert np.array_equal(sc[unr].view(np.uint32), sc2[unr].view(np.uint32))
    assert np.all(nx[unr] == workloads.STATE_UNRESTRICTED)


def test_decode_tail_dfa_advance_matches_arcs_and_dense_table():
    w = workloads.config(4, seed=4, scale_vocab=5000, scale_rows=16)
    tok_a, _, nx_a = oracle.decode_tail(w.x, w.norm_weight, w.epsilon, w.embedding,
                                        w.row_state, w.state_offsets, w.state_tokens,
                                        state_next=w.state_next)
    tok_d, _, nx_d = oracle.decode_tail(w.x, w.norm_weight, w.epsilon, w.embedding,
                                        w.row_state, w.state_offsets, w.state_tokens,
                                        next_table=w.next_table)
    assert np.array_equal(tok_a, tok_d) and np.array_equal(nx_a, nx_d)
    for r in range(w.rows):
        assert nx_d[r] == w.next_table[w.row_state[r], tok_d[r]]


def test_decode_tail_threads_do_not_change_bits():
    w = workloads.config(3, seed=1, scale_vocab=3000, scale_rows=30)
    a = oracle.decode_tail(w.x, w.norm_weight, w.epsilon, w.embedding, w.row_state,
                           w.state_offsets, w.state_tokens, threads=1)
    b = oracle.decode_tail(w.x, w.norm_weight, w.epsilon, w.embedding, w.row_state,
                           w.state_offsets, w.state_tokens, threads=7)
    for u, v in zip(a, b):
        assert np.array_equal(u.view(np.uint32), v.view(np.uint32))


def test_cfg1_single_sequence_full_vocab_vs_reference_linear():
    """FP32 table; the restricted token equals the argmax of the
    reference linear_f32 logits over the allowed ids, and the full-vocabulary
    argmax of the same logits equals the oracle's unrestricted row."""
    r = needs_ref()
    w = workloads.config(1, seed=0)
    y = oracle.rms_norm_f32(w.x, w.norm_weight, w.epsilon)
    logits = np.empty((1, w.vocab), np.float32)
    assert r.mfref_linear_f32(y.ctypes.data, w.embedding.ctypes.data,
                              logits.ctypes.data, 1, w.hidden, w.vocab) == 0
    tok, sc, _ = oracle.decode_tail(w.x, w.norm_weight, w.epsilon, w.embedding,
                                    w.row_state, w.state_offsets, w.state_tokens,
                                    order=oracle.ORDER_MUL_ADD_CHAIN)
    ids = w.state_tokens
    v = logits[0, ids]
    assert tok[0] == ids[v == v.max()].min() and sc[0] == v.max()
    unr = np.array([workloads.STATE_UNRESTRICTED], np.uint32)
    ftok, fsc, _ = oracle.decode_tail(w.x, w.norm_weight, w.epsilon, w.embedding,
                                      unr, w.state_offsets, w.state_tokens,
                                      order=oracle.ORDER_MUL_ADD_CHAIN, threads=8)
    assert ftok[0] == int(np.argmax(logits[0])) and fsc[0] == logits[0].max()
