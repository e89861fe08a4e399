"""Token DFAs on the host, and their device export.

``TokenDfa`` keeps the reference grammar layer's interface and rules
(include/marketforge/grammar/token_dfa.hpp:15-74, src/grammar/token_dfa.cpp):
a prefix-free token trie over a finite set of choices, states numbered in
creation order, each state's arcs ascending by token, ``advance`` by binary
search, and a terminal state per choice.  ``ActionDfa``
(src/grammar/action_dfa.cpp:30-109) builds the same trie over market actions,
so its states and arcs come out identical for the same token sequences.

``DfaTables`` is the export the decode tail consumes: CSR offsets / arc
tokens / arc next states (the per-state ``allowed`` spans,
token_dfa.cpp:100-109, laid end to end) plus each state's terminal choice.
``DfaTables.from_dfa`` uses only the public queries (``state_count``,
``allowed``, ``terminal``, ``decode_terminal``), so it exports any object with
the reference's interface.
"""
from __future__ import annotations

import bisect
from dataclasses import dataclass
from typing import List, Optional, Sequence, Tuple

import numpy as np

NO_CHOICE = 0xFFFFFFFF

# reference ErrorCode values (include/marketforge/core/status.hpp)
INVALID_ARGUMENT = 1
INVALID_FORMAT = 11
RESOURCE_LIMIT = 15


class DfaError(ValueError):
    """A failed grammar call; ``code`` is the reference ErrorCode."""

    def __init__(self, code: int, what: str):
        super().__init__(f"{what} (error code {code})")
        self.code = code


@dataclass(frozen=True)
class DfaConfig:
    """TokenDfaConfig (token_dfa.hpp:21-27)."""
    vocabulary_size: int
    maximum_sequence_tokens: int = 32
    maximum_choices: int = 4096
    maximum_states: int = 65536
    maximum_arcs: int = 65536


class TokenDfa:
    """A deterministic token trie over finite choices (token_dfa.hpp:30-74)."""

    def __init__(self, first_arc: List[int], arc_count: List[int], terminal: List[int],
                 arc_tokens: List[int], arc_next: List[int], choices: List[int]):
        self._first = first_arc
        self._count = arc_count
        self._terminal = terminal          # index into choices, or NO_CHOICE
        self._tokens = arc_tokens
        self._next = arc_next
        self._choices = choices

    @staticmethod
    def build(language: Sequence[Tuple[int, Sequence[int]]], config: DfaConfig) -> "TokenDfa":
        """``language``: (choice id, token sequence) pairs.  Raises DfaError
        with the reference's codes (token_dfa.cpp:23-95): invalid_argument for
        an empty language or config field, a repeated or reserved choice id,
        an empty, too long or out-of-vocabulary sequence, or one that is a
        prefix of another; resource_limit past the configured counts."""
        if (not language or config.vocabulary_size == 0 or config.maximum_sequence_tokens == 0
                or config.maximum_choices == 0 or config.maximum_states == 0
                or config.maximum_arcs == 0):
            raise DfaError(INVALID_ARGUMENT, "empty language or zero limit")
        if len(language) > config.maximum_choices:
            raise DfaError(RESOURCE_LIMIT, "more choices than maximum_choices")
        children: List[dict] = [{}]
        ends: List[int] = [NO_CHOICE]     # choice index ending at each node
        choices: List[int] = []
        seen = set()
        arcs = 0
        for cid, seq in language:
            seq = [int(t) for t in seq]
            if cid == NO_CHOICE or not seq or len(seq) > config.maximum_sequence_tokens \
                    or cid in seen:
                raise DfaError(INVALID_ARGUMENT, f"choice {cid}: bad id or sequence")
            seen.add(cid)
            node = 0
            for t in seq:
                if t >= config.vocabulary_size or ends[node] != NO_CHOICE:
                    raise DfaError(INVALID_ARGUMENT, f"choice {cid}: token {t} or prefix")
                nxt = children[node].get(t)
                if nxt is None:
                    if len(children) >= config.maximum_states or arcs >= config.maximum_arcs:
                        raise DfaError(RESOURCE_LIMIT, "more states or arcs than the limits")
                    nxt = len(children)
                    children[node][t] = nxt
                    children.append({})
                    ends.append(NO_CHOICE)
                    arcs += 1
                node = nxt
            if ends[node] != NO_CHOICE or children[node]:
                raise DfaError(INVALID_ARGUMENT, f"choice {cid}: repeats or prefixes another")
            ends[node] = len(choices)
            choices.append(int(cid))
        first, count, tokens, nexts = [], [], [], []
        for node in range(len(children)):
            first.append(len(tokens))
            count.append(len(children[node]))
            for t in sorted(children[node]):
                tokens.append(t)
                nexts.append(children[node][t])
        if len(tokens) != arcs or len(choices) != len(language):
            raise DfaError(INVALID_FORMAT, "inconsistent trie")
        return TokenDfa(first, count, ends, tokens, nexts, choices)

    def root(self) -> int:
        return 0

    def state_count(self) -> int:
        return len(self._first)

    def arc_count(self) -> int:
        return len(self._tokens)

    def choice_count(self) -> int:
        return len(self._choices)

    def _check(self, state: int) -> None:
        if not 0 <= state < len(self._first):
            raise DfaError(INVALID_ARGUMENT, f"state {state} out of range")

    def allowed(self, state: int) -> List[Tuple[int, int]]:
        """The state's arcs as (token, next state), ascending by token."""
        self._check(state)
        b = self._first[state]
        e = b + self._count[state]
        return list(zip(self._tokens[b:e], self._next[b:e]))

    def advance(self, state: int, token: int) -> int:
        """token_dfa.cpp:111-128: lower_bound over the state's arcs."""
        self._check(state)
        b = self._first[state]
        e = b + self._count[state]
        i = bisect.bisect_left(self._tokens, token, b, e)
        if i == e or self._tokens[i] != token:
            raise DfaError(INVALID_ARGUMENT, f"token {token} not allowed in state {state}")
        return self._next[i]

    def terminal(self, state: int) -> bool:
        return 0 <= state < len(self._first) and self._terminal[state] != NO_CHOICE

    def decode_terminal(self, state: int) -> int:
        self._check(state)
        k = self._terminal[state]
        if k == NO_CHOICE:
            raise DfaError(INVALID_ARGUMENT, f"state {state} is not terminal")
        return self._choices[k]


@dataclass
class DfaTables:
    """The device export of a token DFA.

    offsets u32[S + 1], tokens u32[A], next u32[A]: the CSR lists the decode
    tail reads (``state_offsets``, ``state_tokens``, ``state_next``);
    choice u32[S]: the terminal choice of each state (NO_CHOICE otherwise);
    max_count: the longest list; depth: the most tokens on a path from the
    root to a terminal state (the steps a decode loop needs)."""
    offsets: np.ndarray
    tokens: np.ndarray
    next: np.ndarray
    choice: np.ndarray
    max_count: int
    depth: int

    @property
    def states(self) -> int:
        return int(self.offsets.size - 1)

    @property
    def arcs(self) -> int:
        return int(self.tokens.size)

    @staticmethod
    def from_dfa(dfa) -> "DfaTables":
        """Export through the reference's public DFA queries."""
        S = dfa.state_count()
        offsets = np.zeros(S + 1, np.uint32)
        tokens: List[int] = []
        nexts: List[int] = []
        choice = np.full(S, NO_CHOICE, np.uint32)
        for s in range(S):
            offsets[s] = len(tokens)
            for t, n in dfa.allowed(s):
                tokens.append(t)
                nexts.append(n)
            if dfa.terminal(s):
                choice[s] = dfa.decode_terminal(s)
        offsets[S] = len(tokens)
        return DfaTables.from_arrays(offsets, np.asarray(tokens, np.uint32),
                                     np.asarray(nexts, np.uint32), choice)

    @staticmethod
    def from_arrays(offsets, tokens, nexts, choice=None, vocab: Optional[int] = None) -> "DfaTables":
        """Checks CSR arrays (monotone offsets, strictly ascending tokens per
        state, next states in range, tokens below ``vocab``) and computes
        max_count and depth.  Raises DfaError(invalid_format)."""
        o = np.ascontiguousarray(offsets, dtype=np.uint32)
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        n = np.ascontiguousarray(nexts, dtype=np.uint32)
        S = o.size - 1
        if S < 1 or o[0] != 0 or o[-1] != t.size or t.size != n.size:
            raise DfaError(INVALID_FORMAT, "offsets do not frame the arcs")
        deg = np.diff(o.astype(np.int64))
        if np.any(deg < 0):
            raise DfaError(INVALID_FORMAT, "offsets decrease")
        if t.size and int(n.max()) >= S:
            raise DfaError(INVALID_FORMAT, "a next state is out of range")
        if vocab is not None and t.size and int(t.max()) >= vocab:
            raise DfaError(INVALID_FORMAT, "a token is outside the vocabulary")
        same_state = np.repeat(np.arange(S), deg)
        if t.size > 1 and np.any((np.diff(t.astype(np.int64)) <= 0)
                                 & (same_state[1:] == same_state[:-1])):
            raise DfaError(INVALID_FORMAT, "tokens of a state are not strictly ascending")
        if choice is None:
            choice = np.full(S, NO_CHOICE, np.uint32)
        choice = np.ascontiguousarray(choice, dtype=np.uint32)
        if choice.size != S:
            raise DfaError(INVALID_FORMAT, "one choice entry per state expected")
        return DfaTables(o, t, n, choice, int(deg.max()) if S else 0, _depth(o, n))

    def advance(self, state: int, token: int) -> int:
        """The arc of ``token`` from ``state`` (token_dfa.cpp:111-128)."""
        b, e = int(self.offsets[state]), int(self.offsets[state + 1])
        i = b + int(np.searchsorted(self.tokens[b:e], token))
        if i == e or int(self.tokens[i]) != token:
            raise DfaError(INVALID_ARGUMENT, f"token {token} not allowed in state {state}")
        return int(self.next[i])


def _depth(offsets: np.ndarray, nexts: np.ndarray) -> int:
    """Longest arc path from the root (a trie: every state has one parent,
    children are numbered after their parent in trie builds, but any acyclic
    export is handled by a breadth-first walk bounded by the state count)."""
    S = offsets.size - 1
    level = {0}
    depth = 0
    seen = 0
    while level:
        nxt = set()
        for s in level:
            nxt.update(int(v) for v in nexts[offsets[s]:offsets[s + 1]])
        seen += 1
        if not nxt:
            break
        if seen > S:
            raise DfaError(INVALID_FORMAT, "the DFA has a cycle")
        depth += 1
        level = nxt
    return depth


# Binary form read by the C++ tools (market_sim_amd/bench): little-endian u32
# magic "MFD1", states S, arcs A, then offsets[S + 1], tokens[A], next[A],
# choice[S].
_MAGIC = 0x3144464D


def write_tables(tables: DfaTables, path: str) -> None:
    head = np.array([_MAGIC, tables.states, tables.arcs], np.uint32)
    with open(path, "wb") as f:
        for a in (head, tables.offsets, tables.tokens, tables.next, tables.choice):
            f.write(np.ascontiguousarray(a, dtype="<u4").tobytes())


def read_tables(path: str) -> DfaTables:
    raw = np.fromfile(path, dtype="<u4")
    if raw.size < 3 or raw[0] != _MAGIC:
        raise DfaError(INVALID_FORMAT, f"{path}: not a DFA table file")
    S, A = int(raw[1]), int(raw[2])
    if raw.size != 3 + (S + 1) + 2 * A + S:
        raise DfaError(INVALID_FORMAT, f"{path}: truncated")
    o = raw[3:4 + S]
    t = raw[4 + S:4 + S + A]
    n = raw[4 + S + A:4 + S + 2 * A]
    c = raw[4 + S + 2 * A:]
    return DfaTables.from_arrays(o, t, n, c)
