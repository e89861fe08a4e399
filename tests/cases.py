"""Inputs of the reference's own tests for this path, restated as numpy data.

Each builder cites the reference test it restates.  CPU tests run them through
the oracle; GPU tests run the same inputs through the HIP library, so both
sides see identical bytes.
"""
import math
import os

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
INVALID = 0xFFFFFFFF


def f16_bits(values) -> np.ndarray:
    return np.asarray(values, np.float32).astype(np.float16).view(np.uint16)


def tiny_head_case():
    """tests/cuda/cuda_tests.cu:699-735: rows=3, H=8, V=17, max_allowed=5.

    Embedding row 6 duplicates row 4 (a tie) and hidden row 2 is all NaN."""
    rows, hidden, vocab, max_allowed = 3, 8, 17, 5
    allowed = np.array([9, 3, 14, 0, 0, 6, 4, 8, 0, 0, 7, 1, 0, 0, 0], np.uint32)
    counts = np.array([3, 3, 2], np.uint32)
    h = np.array([((i % 11) - 5) / 8.0 for i in range(rows * hidden)], np.float32)
    e = np.array([(((i * 7) % 19) - 9) / 16.0 for i in range(vocab * hidden)],
                 np.float32)
    e = e.reshape(vocab, hidden)
    h = h.reshape(rows, hidden)
    e[6] = e[4]
    h[2] = np.nan
    return dict(hidden=f16_bits(h), embedding=f16_bits(e), allowed=allowed,
                counts=counts, rows=rows, hidden_size=hidden, vocab=vocab,
                max_allowed=max_allowed)


def greedy_case(rows: int, vocab: int):
    """tests/cuda/cuda_tests.cu:508-531: winner (row*7+3)%V; row 1 ties 9 and
    its winner; row 2 is all -inf with a NaN at token 0 -> token 1."""
    logits = np.full((rows, vocab), -4.0, np.float32)
    expected = np.zeros(rows, np.uint32)
    for r in range(rows):
        w = (r * 7 + 3) % vocab
        expected[r] = w
        logits[r, w] = 8.0
    if rows > 1 and vocab > 9:
        logits[1, 9] = 8.0
        expected[1] = 9
    if rows > 2 and vocab > 1:
        logits[2, :] = -np.inf
        logits[2, 0] = np.nan
        expected[2] = 1
    return f16_bits(logits), expected


def market_dfa():
    d = np.load(os.path.join(GOLDEN, "market_dfa.npz"))
    return d["offsets"], d["tokens"], d["next"]


def market_dfa_terminal():
    """Per state, the index of its terminal action among the catalog's
    entries (0xFFFFFFFF: not terminal)."""
    return np.load(os.path.join(GOLDEN, "market_dfa.npz"))["terminal"]


def market_language():
    """The catalog's entries as token sequences, in catalog order."""
    d = np.load(os.path.join(GOLDEN, "market_dfa.npz"))
    o, t = d["language_offsets"], d["language_tokens"]
    return [t[o[i]:o[i + 1]].tolist() for i in range(o.size - 1)]


def market_restricted_greedy_case():
    """tests/cuda/cuda_tests.cu:567-651: the first 8 non-empty market-DFA
    states; row 0 all 4.0 (lowest id wins), row 1 all NaN (lowest id), other
    rows (token*17+row)%31; a disallowed token carries 100.0 and must lose."""
    offsets, tokens, _ = market_dfa()
    vocab = 49152
    rows_lists = []
    for s in range(len(offsets) - 1):
        if len(rows_lists) == 8:
            break
        if offsets[s + 1] > offsets[s]:
            rows_lists.append(tokens[offsets[s]:offsets[s + 1]].copy())
    rows = len(rows_lists)
    max_allowed = max(len(c) for c in rows_lists)
    logits = np.full((rows, vocab), -8.0, np.float32)
    allowed = np.full((rows, max_allowed), INVALID, np.uint32)
    counts = np.zeros(rows, np.uint32)
    for r, cands in enumerate(rows_lists):
        counts[r] = len(cands)
        disallowed = vocab - 1
        while disallowed in set(cands.tolist()):
            disallowed -= 1
        logits[r, disallowed] = 100.0
        for i, t in enumerate(cands):
            allowed[r, i] = t
            if r == 0:
                v = 4.0
            elif r == 1:
                v = math.nan
            else:
                v = float((int(t) * 17 + r) % 31)
            logits[r, t] = v
    return dict(logits=f16_bits(logits), allowed=allowed, counts=counts,
                rows=rows, vocab=vocab, max_allowed=max_allowed,
                lists=rows_lists)


def invalid_rows_greedy_case():
    """tests/cuda/cuda_tests.cu:1173-1255: count 0, count > max, id >= V."""
    vocab, max_allowed = 8, 4
    logits = f16_bits(np.zeros((1, vocab), np.float32))
    return [
        (logits, np.array([[1, 3, 5, 7]], np.uint32), np.array([0], np.uint32)),
        (logits, np.array([[1, 3, 5, 7]], np.uint32), np.array([5], np.uint32)),
        (logits, np.array([[1, 8, 5, 7]], np.uint32), np.array([2], np.uint32)),
    ], vocab, max_allowed


def invalid_rows_head_case():
    """tests/cuda/cuda_tests.cu:1341-1403: counts {0, 3 > max, 2 with id 5 >= V}."""
    rows, hidden, vocab, max_allowed = 3, 2, 5, 2
    return dict(hidden=f16_bits(np.zeros((rows, hidden))),
                embedding=f16_bits(np.zeros((vocab, hidden))),
                allowed=np.array([1, 2, 2, 3, 1, 5], np.uint32),
                counts=np.array([0, 3, 2], np.uint32), rows=rows,
                hidden_size=hidden, vocab=vocab, max_allowed=max_allowed)


def rms_norm_case(rows: int, hidden: int):
    """tests/cuda/cuda_tests.cu:63-77 input pattern."""
    n = rows * hidden
    x = np.array([((i % 37) - 18) * 0.0625 for i in range(n)], np.float32)
    w = np.array([0.75 + (i % 17) * 0.03125 for i in range(hidden)], np.float32)
    return x.reshape(rows, hidden), w


RMS_SHAPES = [(2, 1), (3, 255), (3, 256), (3, 257), (7, 576), (2, 1024)]


def linear_case(rows: int, inf: int, outf: int):
    """tests/cuda/cuda_tests.cu:144-181 input pattern."""
    x = np.array([((i % 17) - 8) / 32.0 for i in range(rows * inf)], np.float32)
    w = np.array([((i % 13) - 6) / 64.0 for i in range(outf * inf)], np.float32)
    return f16_bits(x.reshape(rows, inf)), f16_bits(w.reshape(outf, inf))


def real_logits():
    """tests/fixtures/golden/smollm2-pr4-greedy-f32.*: SmolLM2-135M FP32 logits
    [3, 49152] with expected tokens [198, 198, 504]."""
    from safetensors.numpy import load_file
    d = load_file(os.path.join(GOLDEN, "smollm2-pr4-greedy-f32.safetensors"))
    return (d["expected.logits"], d["expected.tokens"].astype(np.uint32),
            d["expected.margins"])


# src/tools/cuda_smollm2_conformance.cu:85-107 legal sets for the three rows.
REAL_LEGAL_SETS = [[42, 198, 504, 900], [17, 198, 504, 777], [3, 198, 504, 1024]]
