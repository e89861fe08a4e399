"""The host token DFA and its device export (market_sim_amd/dfa.py).

Pinned by the reference's own unit cases (tests/unit/token_dfa_tests.cpp),
by the reference's TokenDfa built from its sources (oracle/_ref, where it is
built) on random languages, and by the real SmolLM2 market-action DFA the
reference builds (tests/golden/market_dfa.npz).
"""
import ctypes

import numpy as np
import pytest

import oracle
from market_sim_amd import dfa as D
from tests import cases

CONFIG = D.DfaConfig(64, 8, 16, 32, 32)   # token_dfa_tests.cpp:18-20


def test_builds_generic_choices_and_decodes_terminal_ids():
    # token_dfa_tests.cpp:22-49
    d = D.TokenDfa.build([(41, [9, 4]), (7, [3, 8, 1]), (99, [9, 6])], CONFIG)
    assert (d.choice_count(), d.state_count(), d.arc_count()) == (3, 7, 6)
    assert [t for t, _ in d.allowed(d.root())] == [3, 9]
    s = d.advance(d.advance(d.root(), 9), 6)
    assert d.terminal(s) and d.decode_terminal(s) == 99


@pytest.mark.parametrize("language", [
    [(1, [2]), (1, [3])],          # duplicate ids
    [(1, [2]), (2, [2, 3])],       # prefix collision
    [(2, [2, 3]), (1, [2])],       # prefix collision, other order
    [(1, [64])],                   # token outside the vocabulary
    [(0xFFFFFFFF, [1])],           # reserved id
    [(1, [])],                     # empty sequence
    [(1, list(range(9)))],         # longer than maximum_sequence_tokens
    [],                            # empty language
])
def test_rejects_ambiguous_or_invalid_languages(language):
    # token_dfa_tests.cpp:51-76
    with pytest.raises(D.DfaError) as e:
        D.TokenDfa.build(language, CONFIG)
    assert e.value.code == D.INVALID_ARGUMENT


def test_enforces_explicit_resource_limits():
    # token_dfa_tests.cpp:78-97
    lang = [(1, [1, 2]), (2, [3, 4])]
    with pytest.raises(D.DfaError) as e:
        D.TokenDfa.build(lang, D.DfaConfig(64, 8, 16, 2, 32))
    assert e.value.code == D.RESOURCE_LIMIT
    with pytest.raises(D.DfaError) as e:
        D.TokenDfa.build(lang, D.DfaConfig(64, 8, 1, 32, 32))
    assert e.value.code == D.RESOURCE_LIMIT
    d = D.TokenDfa.build(lang, CONFIG)
    for call in (lambda: d.allowed(99), lambda: d.advance(d.root(), 63),
                 lambda: d.decode_terminal(d.root())):
        with pytest.raises(D.DfaError) as e:
            call()
        assert e.value.code == D.INVALID_ARGUMENT


def _random_language(rng, n, vocab, max_len):
    """n distinct prefix-free token sequences (a random trie's leaves)."""
    out, seqs = [], set()
    while len(out) < n:
        seq = tuple(int(t) for t in rng.integers(0, vocab, rng.integers(1, max_len + 1)))
        if any(seq[:k] in seqs for k in range(1, len(seq) + 1)) or \
                any(s[:len(seq)] == seq for s in seqs):
            continue
        seqs.add(seq)
        out.append((int(rng.integers(0, 1 << 30)) * 2 + len(out) % 2, list(seq)))
    ids = [c for c, _ in out]
    return out if len(set(ids)) == len(ids) else _random_language(rng, n, vocab, max_len)


@pytest.mark.parametrize("seed", range(6))
def test_export_matches_the_reference_build(seed):
    r = oracle.ref()
    if r is None:
        pytest.skip("oracle/_ref (the reference's CPU build) is not built")
    rng = np.random.default_rng(seed)
    lang = _random_language(rng, int(rng.integers(1, 60)), 40 + 20 * seed, 6)
    cfg = D.DfaConfig(40 + 20 * seed, 8, 4096, 65536, 65536)
    tab = D.DfaTables.from_dfa(D.TokenDfa.build(lang, cfg))
    ids = np.array([c for c, _ in lang], np.uint32)
    offs = np.zeros(len(lang) + 1, np.uint32)
    offs[1:] = np.cumsum([len(s) for _, s in lang])
    toks = np.array([t for _, s in lang for t in s], np.uint32)
    cap = 1024
    o = np.zeros(cap, np.uint32); t = np.zeros(cap, np.uint32)
    n = np.zeros(cap, np.uint32); term = np.zeros(cap, np.uint32)
    ns, na = ctypes.c_uint32(), ctypes.c_uint32()
    rc = r.mfref_token_dfa_export(ids.ctypes.data, offs.ctypes.data, toks.ctypes.data,
                                  len(lang), cfg.vocabulary_size, 8, 4096, 65536, 65536,
                                  o.ctypes.data, t.ctypes.data, n.ctypes.data,
                                  term.ctypes.data, cap, cap, ctypes.byref(ns),
                                  ctypes.byref(na))
    assert rc == 0
    assert np.array_equal(tab.offsets, o[:ns.value + 1])
    assert np.array_equal(tab.tokens, t[:na.value]) and np.array_equal(tab.next, n[:na.value])
    assert np.array_equal(tab.choice, term[:ns.value])


def test_real_market_grammar_rebuilds_the_reference_dfa():
    """The catalog's 1585 entries (choice id = entry index) rebuild the
    reference's market-action DFA arc for arc, with the same terminals."""
    lang = list(enumerate(cases.market_language()))
    d = D.TokenDfa.build(lang, D.DfaConfig(49152, 12, 4096, 65536, 65536))
    tab = D.DfaTables.from_dfa(d)
    offsets, tokens, nxt = cases.market_dfa()
    assert np.array_equal(tab.offsets, offsets)
    assert np.array_equal(tab.tokens, tokens) and np.array_equal(tab.next, nxt)
    assert np.array_equal(tab.choice, cases.market_dfa_terminal())
    assert tab.max_count == 11 and tab.states == 3230 and tab.arcs == 3229
    # every entry round-trips: its tokens lead from the root to its terminal
    for i, seq in lang[::37]:
        s = 0
        for tok in seq:
            s = tab.advance(s, tok)
        assert tab.choice[s] == i
    assert tab.depth == max(len(seq) for _, seq in lang)


def test_from_arrays_rejects_malformed_tables():
    o, t, n = np.array([0, 2, 2, 2]), np.array([5, 3]), np.array([1, 2])
    for args in [(o, t, n),                                         # not ascending
                 (np.array([0, 2, 1, 2]), np.array([3, 5]), n),    # offsets decrease
                 (o, np.array([3, 5]), np.array([1, 3])),          # next out of range
                 (np.array([1, 2, 2, 2]), np.array([3, 5]), n)]:   # first offset
        with pytest.raises(D.DfaError):
            D.DfaTables.from_arrays(*args)
    with pytest.raises(D.DfaError):
        D.DfaTables.from_arrays(o, np.array([3, 5]), n, vocab=5)
    ok = D.DfaTables.from_arrays(o, np.array([3, 5]), n)
    assert (ok.max_count, ok.depth, ok.states) == (2, 1, 3)
