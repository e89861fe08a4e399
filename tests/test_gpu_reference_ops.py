"""GPU parity of the reference operators (greedy.hpp, rms_norm.hpp, linear.hpp)
against the CPU oracle, through the C ABI.  Restates the reference's own GPU
tests (tests/cuda/cuda_tests.cu) with identical inputs."""
import math

import numpy as np
import pytest

import oracle
from tests import cases
from tests.gpu_util import B, dev, empty, host, ok, stream

pytestmark = pytest.mark.gpu
INVALID = cases.INVALID


@pytest.fixture(autouse=True)
def _lib(hip):
    return hip


# ------------------------------------------------------------ greedy -------

@pytest.mark.parametrize("rows,vocab", [(1, 17), (3, 49152)])
def test_greedy_f16_lowest_id_tie_rule(rows, vocab):
    """cuda_tests.cu:1132-1135."""
    from market_sim_amd import ops
    logits, expected = cases.greedy_case(rows, vocab)
    out = empty(rows, np.uint32)
    ld = dev(logits)
    ok(ops.greedy_select_f16(B(ld), B(out), rows, vocab, stream()))
    got = host(out, np.uint32)
    assert got.tolist() == expected.tolist() == oracle.greedy_f16(logits).tolist()


def test_greedy_f32_real_smollm2_logits():
    from market_sim_amd import ops
    logits, tokens, _ = cases.real_logits()
    out = empty(3, np.uint32)
    ld = dev(logits)
    ok(ops.greedy_select_f32(B(ld), B(out), 3, 49152, stream()))
    assert host(out, np.uint32).tolist() == [198, 198, 504]


def test_greedy_f16_all_nan_row_selects_zero_and_random_rows():
    from market_sim_amd import ops
    rng = np.random.default_rng(5)
    logits = rng.standard_normal((9, 1000)).astype(np.float16)
    logits[3] = np.nan
    logits[4, ::7] = logits[4].max()  # many exact ties
    bits = logits.view(np.uint16)
    out = empty(9, np.uint32)
    ld = dev(bits)
    ok(ops.greedy_select_f16(B(ld), B(out), 9, 1000, stream()))
    assert host(out, np.uint32).tolist() == oracle.greedy_f16(bits).tolist()


def test_restricted_greedy_f16_market_dfa():
    """cuda_tests.cu:1169-1171 (market-action DFA states)."""
    from market_sim_amd import ops
    c = cases.market_restricted_greedy_case()
    out = empty(c["rows"], np.uint32)
    ld, ad, cd = dev(c["logits"]), dev(c["allowed"]), dev(c["counts"])
    ok(ops.restricted_greedy_select_f16(B(ld), B(ad), B(cd), B(out), c["rows"],
                                        c["vocab"], c["max_allowed"], stream()))
    expected = oracle.restricted_greedy_f16(c["logits"], c["allowed"], c["counts"],
                                            c["max_allowed"])
    assert host(out, np.uint32).tolist() == expected.tolist()


def test_restricted_greedy_invalid_device_rows():
    """cuda_tests.cu:1173-1255."""
    from market_sim_amd import ops
    variants, vocab, max_allowed = cases.invalid_rows_greedy_case()
    for logits, allowed, counts in variants:
        out = empty(1, np.uint32)
        ld, ad, cd = dev(logits), dev(allowed), dev(counts)
        ok(ops.restricted_greedy_select_f16(B(ld), B(ad), B(cd), B(out), 1, vocab,
                                            max_allowed, stream()))
        assert host(out, np.uint32).tolist() == [INVALID]


def test_restricted_greedy_f32_real_logits_legal_sets():
    """src/tools/cuda_smollm2_conformance.cu:85-107 legal sets."""
    from market_sim_amd import ops
    logits, _, _ = cases.real_logits()
    allowed = np.array(cases.REAL_LEGAL_SETS, np.uint32)
    counts = np.full(3, 4, np.uint32)
    out = empty(3, np.uint32)
    ld, ad, cd = dev(logits), dev(allowed), dev(counts)
    ok(ops.restricted_greedy_select_f32(B(ld), B(ad), B(cd), B(out), 3, 49152, 4, stream()))
    assert host(out, np.uint32).tolist() == [198, 198, 504]


# ---------------------------------------------------- restricted head f16 ---

def _run_head(c):
    from market_sim_amd import ops
    out = empty(c["rows"], np.uint32)
    keep = [dev(c[k]) for k in ("hidden", "embedding", "allowed", "counts")]
    ok(ops.restricted_output_head_f16(*[B(t) for t in keep], B(out),
                                      c["rows"], c["hidden_size"], c["vocab"],
                                      c["max_allowed"], stream()))
    return host(out, np.uint32)


def test_restricted_output_head_tiny_known_answer():
    """cuda_tests.cu:1279-1281: [14, 8, 1]."""
    assert _run_head(cases.tiny_head_case()).tolist() == [14, 8, 1]


def test_restricted_output_head_invalid_device_rows():
    """cuda_tests.cu:1341-1403."""
    assert _run_head(cases.invalid_rows_head_case()).tolist() == [INVALID] * 3


@pytest.mark.parametrize("hidden,vocab,rows,max_allowed", [
    (576, 49152, 16, 128), (576, 5000, 7, 3000), (64, 3000, 5, 700), (100, 4000, 4, 300)])
def test_restricted_output_head_matches_reference_fma_chain(hidden, vocab, rows, max_allowed):
    """Random FP16 rows, ragged counts, several blocks per row; the tokens
    equal the reference kernel's sequential fmaf chain (greedy.cu:171-176)."""
    rng = np.random.default_rng(hidden + rows)
    h = rng.standard_normal((rows, hidden)).astype(np.float16).view(np.uint16)
    e = (rng.standard_normal((vocab, hidden)) * 0.02).astype(np.float16).view(np.uint16)
    allowed = np.zeros((rows, max_allowed), np.uint32)
    counts = rng.integers(1, max_allowed + 1, rows).astype(np.uint32)
    for r in range(rows):
        allowed[r, :counts[r]] = rng.choice(vocab, counts[r], replace=False)
    c = dict(hidden=h, embedding=e, allowed=allowed, counts=counts, rows=rows,
             hidden_size=hidden, vocab=vocab, max_allowed=max_allowed)
    expected, _ = oracle.restricted_output_head_f16(h, e, allowed, counts, max_allowed)
    assert _run_head(c).tolist() == expected.tolist()


def test_restricted_output_head_wide_hidden_and_long_lists():
    """Shapes past the LDS staging of the hidden row (H > 16384: read from
    global memory) and past one LDS array of block records (more than
    256 x 1024 candidates: the records are merged in stages); the reference
    runs both (greedy.cu:355-399 caps only at 32-bit sizes)."""
    rng = np.random.default_rng(23)
    # wide hidden: 16448 features, a few hundred candidates per row
    hidden, vocab, rows, max_allowed = 16448, 700, 3, 400
    h = rng.standard_normal((rows, hidden)).astype(np.float16).view(np.uint16)
    e = (rng.standard_normal((vocab, hidden)) * 0.02).astype(np.float16).view(np.uint16)
    allowed = np.zeros((rows, max_allowed), np.uint32)
    counts = np.array([400, 1, 257], np.uint32)
    for r in range(rows):
        allowed[r, :counts[r]] = rng.choice(vocab, counts[r], replace=False)
    c = dict(hidden=h, embedding=e, allowed=allowed, counts=counts, rows=rows,
             hidden_size=hidden, vocab=vocab, max_allowed=max_allowed)
    expected, _ = oracle.restricted_output_head_f16(h, e, allowed, counts, max_allowed)
    assert _run_head(c).tolist() == expected.tolist()
    # long lists: 300,000 candidates (ids repeat) over a small vocabulary,
    # one row with the best id near the end of its list
    hidden, vocab, rows, max_allowed = 64, 4096, 2, 300_000
    h = rng.standard_normal((rows, hidden)).astype(np.float16).view(np.uint16)
    e = (rng.standard_normal((vocab, hidden)) * 0.02).astype(np.float16).view(np.uint16)
    allowed = rng.integers(0, vocab, (rows, max_allowed)).astype(np.uint32)
    counts = np.array([max_allowed, 270_001], np.uint32)
    c = dict(hidden=h, embedding=e, allowed=allowed, counts=counts, rows=rows,
             hidden_size=hidden, vocab=vocab, max_allowed=max_allowed)
    expected, _ = oracle.restricted_output_head_f16(h, e, allowed, counts, max_allowed)
    assert _run_head(c).tolist() == expected.tolist()


def test_restricted_output_head_near_ties_are_exact():
    """Candidates whose scores differ only in the last bits: embedding rows
    that are permutations of one another give equal exact sums, so only the
    reference order's rounding separates them."""
    rng = np.random.default_rng(17)
    hidden, vocab, rows = 576, 400, 6
    base = (rng.standard_normal(hidden) * 0.02).astype(np.float16)
    e = np.stack([rng.permutation(base) for _ in range(vocab)]).view(np.uint16)
    h = np.ones((rows, hidden), np.float16)
    h[:, : hidden // 2] = rng.standard_normal((rows, hidden // 2)).astype(np.float16)
    h = h.view(np.uint16)
    allowed = np.tile(np.arange(vocab, dtype=np.uint32)[None, :256], (rows, 1))
    counts = np.full(rows, 256, np.uint32)
    c = dict(hidden=h, embedding=e, allowed=allowed, counts=counts, rows=rows,
             hidden_size=hidden, vocab=vocab, max_allowed=256)
    expected, _ = oracle.restricted_output_head_f16(h, e, allowed, counts, 256)
    assert _run_head(c).tolist() == expected.tolist()


# ------------------------------------------------------------- RMSNorm -----

@pytest.mark.parametrize("rows,hidden", cases.RMS_SHAPES)
def test_rms_norm_f32_bit_exact_vs_cpu_oracle(rows, hidden):
    """cuda_tests.cu:905-912 shapes; bit-exact (the reference allows 3e-5)."""
    from market_sim_amd import ops
    x, w = cases.rms_norm_case(rows, hidden)
    in_place = hidden == 1024
    xd, wd = dev(x), dev(w)
    out = xd if in_place else empty(rows * hidden, np.float32)
    ok(ops.rms_norm_f32(B(xd), B(wd), B(out), rows, hidden, 1e-5, stream()))
    got = host(out, np.float32).reshape(rows, hidden)
    assert np.array_equal(got.view(np.uint32), oracle.rms_norm_f32(x, w, 1e-5).view(np.uint32))


def test_rms_norm_f32_random_bit_exact():
    from market_sim_amd import ops
    rng = np.random.default_rng(2)
    for hidden in (576, 2048, 777):
        x = (rng.standard_normal((9, hidden)) * 3).astype(np.float32)
        w = (1 + 0.02 * rng.standard_normal(hidden)).astype(np.float32)
        out = empty(9 * hidden, np.float32)
        xd, wd = dev(x), dev(w)
        ok(ops.rms_norm_f32(B(xd), B(wd), B(out), 9, hidden, 1e-5, stream()))
        got = host(out, np.float32).reshape(9, hidden)
        assert np.array_equal(got, oracle.rms_norm_f32(x, w, 1e-5))


def test_rms_norm_wide_rows_bit_exact():
    """Rows wider than the LDS staging (H > 16384): the squares are staged in
    chunks with one feature-order chain; the reference has no width limit."""
    from market_sim_amd import ops
    rng = np.random.default_rng(5)
    for hidden in (16385, 40000):
        x = (rng.standard_normal((3, hidden)) * 2).astype(np.float32)
        w = (1 + 0.02 * rng.standard_normal(hidden)).astype(np.float32)
        out = empty(3 * hidden, np.float32)
        xd, wd = dev(x), dev(w)
        ok(ops.rms_norm_f32(B(xd), B(wd), B(out), 3, hidden, 1e-5, stream()))
        got = host(out, np.float32).reshape(3, hidden)
        assert np.array_equal(got.view(np.uint32), oracle.rms_norm_f32(x, w, 1e-5).view(np.uint32))
        x16 = x.astype(np.float16).view(np.uint16)
        w16 = w.astype(np.float16).view(np.uint16)
        out16 = empty(3 * hidden, np.uint16)
        xd16, wd16 = dev(x16), dev(w16)
        ok(ops.rms_norm_f16(B(xd16), B(wd16), B(out16), 3, hidden, 1e-5, stream()))
        got16 = host(out16, np.uint16).reshape(3, hidden)
        assert np.array_equal(got16, oracle.rms_norm_f16(x16, w16, 1e-5))


def test_rms_norm_f16_bit_exact():
    from market_sim_amd import ops
    rng = np.random.default_rng(4)
    x = rng.standard_normal((5, 576)).astype(np.float16).view(np.uint16)
    w = (1 + 0.02 * rng.standard_normal(576)).astype(np.float16).view(np.uint16)
    out = empty(5 * 576, np.uint16)
    xd, wd = dev(x), dev(w)
    ok(ops.rms_norm_f16(B(xd), B(wd), B(out), 5, 576, 1e-5, stream()))
    got = host(out, np.uint16).reshape(5, 576)
    assert np.array_equal(got, oracle.rms_norm_f16(x, w, 1e-5))


# -------------------------------------------------------------- linear -----

@pytest.mark.parametrize("rows,inf,outf", [(2, 3, 2), (3, 576, 1536), (37, 576, 300)])
def test_linear_f16_matches_reference_test(rows, inf, outf):
    """cuda_tests.cu:947-950 shapes.  The reference bound is |d| <= 0.015; the
    MFMA path must also be within one FP16 ulp of the sequential-fma oracle
    and the simple path (K % 16 != 0) bit-exact."""
    from market_sim_amd import ops
    x, w = cases.linear_case(rows, inf, outf)
    out = empty(rows * outf, np.uint16)
    xd, wd = dev(x), dev(w)
    ok(ops.linear_f16(B(xd), B(wd), B(out), rows, inf, outf, stream()))
    got = host(out, np.uint16).reshape(rows, outf)
    exp16, exp32 = oracle.linear_f16(x, w)
    g = got.view(np.float16).astype(np.float32)
    assert np.max(np.abs(g - exp32)) <= 0.015
    if inf % 16:
        assert np.array_equal(got, exp16)
    else:
        ulps = np.abs(_ordered(got) - _ordered(exp16))
        assert ulps.max() <= 1


@pytest.mark.parametrize("rows,inf,outf", [(1, 32, 5), (300, 64, 400), (257, 96, 193),
                                           (256, 960, 4800), (512, 128, 192)])
def test_linear_f16_mfma_tiles_random(rows, inf, outf):
    """The MFMA projection over random FP16 data at shapes that cut its
    256-row x 192-token tiles and its 32-feature chunks (one chunk, two,
    three; several row tiles; a partial token tile): every output within
    half an FP16 ulp plus the FP32 accumulation bound 2 H 2^-24 sum |x w|
    of the exact product (float64)."""
    from market_sim_amd import ops
    rng = np.random.default_rng(rows * 7 + inf)
    x = rng.uniform(-1.0, 1.0, (rows, inf)).astype(np.float16)
    w = rng.uniform(-1.0, 1.0, (outf, inf)).astype(np.float16)
    out = empty(rows * outf, np.uint16)
    xd, wd = dev(x.view(np.uint16)), dev(w.view(np.uint16))
    ok(ops.linear_f16(B(xd), B(wd), B(out), rows, inf, outf, stream()))
    got = host(out, np.uint16).reshape(rows, outf).view(np.float16).astype(np.float64)
    x64, w64 = x.astype(np.float64), w.astype(np.float64)
    exact = x64 @ w64.T
    mag = np.abs(x64) @ np.abs(w64).T
    half_ulp = np.spacing(np.maximum(np.abs(got), np.abs(exact)).astype(np.float16)).astype(
        np.float64) / 2
    err = np.abs(got - exact)
    assert np.all(err <= half_ulp + 2.0 * inf * 2.0 ** -24 * mag), float(
        np.max(err - half_ulp))


def _ordered(bits: np.ndarray) -> np.ndarray:
    """FP16 bit patterns mapped to integers that are adjacent for adjacent
    floats across the sign boundary."""
    b = bits.astype(np.int32)
    return np.where(b & 0x8000, -(b & 0x7FFF), b)


@pytest.mark.gpu
def test_reference_output_head_benchmark_tool():
    """The reference's 12-cell output-head benchmark, run by the C++ tool with
    shortened iteration counts: a schema-valid document with token parity
    between the full and the restricted head in every cell."""
    import json
    import os
    import subprocess
    from market_sim_amd import schema
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    tool = os.path.join(root, "market_sim_amd", "bench", "_build", "restricted_output_head_bench")
    assert os.path.exists(tool), "market_sim_amd/bench is not built: run __graft_entry__.build()"
    r = subprocess.run([tool, "--iterations-divisor", "50"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0, r.stderr
    doc = json.loads(r.stdout)
    schema.check_output_head_benchmark(doc)
    assert all(m["exact_token_parity"] for m in doc["measurements"])
