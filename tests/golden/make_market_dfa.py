"""Writes tests/golden/market_dfa.npz from the reference's own market-action DFA.

The reference builds a prefix-free token trie over 1585 SmolLM2 market
actions (src/grammar/smollm2_market_actions.cpp:42-73 over the generated table
src/grammar/generated/smollm2_market_action_v1.inc).  This script runs that
code through oracle/_ref (the reference's CPU sources compiled in place by
oracle/Makefile) and stores the DFA as CSR arrays:

  offsets  uint32[S + 1]   first arc of each state (TokenDfa StateRecord)
  tokens   uint32[A]       arc tokens, strictly ascending per state
  next     uint32[A]       arc next states
  terminal uint32[S]       index of the state's terminal action in the
                           catalog's entries (0xFFFFFFFF: not terminal)
  language_offsets uint32[E + 1], language_tokens uint32[T]
                           the token sequence of each catalog entry
                           (src/grammar/smollm2_market_actions.cpp:42-73)

The fixture is data (the DFA the reference builds), committed so that tests on
machines without the reference tree can use it.  Regenerate with
``python tests/golden/make_market_dfa.py`` after ``make -C oracle ref``.
"""
import ctypes
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle  # noqa: E402


def main() -> None:
    ref = oracle.ref()
    if ref is None:
        raise SystemExit("oracle/_ref not built (make -C oracle ref)")
    cap_states, cap_arcs = 8192, 8192
    offsets = np.zeros(cap_states, np.uint32)
    tokens = np.zeros(cap_arcs, np.uint32)
    nxt = np.zeros(cap_arcs, np.uint32)
    terminal = np.zeros(cap_states, np.uint32)
    n_states = ctypes.c_uint32()
    n_arcs = ctypes.c_uint32()
    rc = ref.mfref_market_dfa_export(offsets.ctypes.data, tokens.ctypes.data,
                                     nxt.ctypes.data, terminal.ctypes.data, cap_states, cap_arcs,
                                     ctypes.byref(n_states), ctypes.byref(n_arcs))
    if rc != 0:
        raise SystemExit(f"export failed: {rc}")
    cap_entries, cap_tokens = 4096, 65536
    lo = np.zeros(cap_entries, np.uint32)
    lt = np.zeros(cap_tokens, np.uint32)
    n_entries = ctypes.c_uint32()
    n_tokens = ctypes.c_uint32()
    rc = ref.mfref_market_language(lo.ctypes.data, lt.ctypes.data, cap_entries, cap_tokens,
                                   ctypes.byref(n_entries), ctypes.byref(n_tokens))
    if rc != 0:
        raise SystemExit(f"language export failed: {rc}")
    s, a = n_states.value, n_arcs.value
    e, t = n_entries.value, n_tokens.value
    np.savez(os.path.join(HERE, "market_dfa.npz"), offsets=offsets[: s + 1],
             tokens=tokens[:a], next=nxt[:a], terminal=terminal[:s],
             language_offsets=lo[: e + 1], language_tokens=lt[:t])
    print(f"states={s} arcs={a} entries={e} language tokens={t}")


if __name__ == "__main__":
    main()
