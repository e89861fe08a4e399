"""Seeded synthetic workloads for the restricted head (the five benchmark configurations cfg1..cfg5).

Generation is deterministic: numpy's PCG64 generator, one independent child
stream per component (``SeedSequence(seed).spawn``), normals from
``Generator.standard_normal`` in float32, FP16 tables by IEEE round-to-nearest
from those float32 values.  Large tables are drawn in fixed row blocks so the
values do not depend on available memory.

Row-state conventions (shared with the C-ABI, include/marketforge_hip.h):
  state < S                 the row is restricted to CSR list ``state``
  STATE_UNRESTRICTED        the row scores the whole vocabulary (MFMA fallback)

For the ragged pack configs (2, 3, 5) every restricted row carries its own
list, so ``state_offsets`` is the per-row CSR and ``row_state[r] == r``.
Lists are sorted ascending with distinct ids, like the arcs of a reference
TokenDfa state (src/grammar/token_dfa.cpp:100-109).
"""
from __future__ import annotations

import dataclasses
import math
from typing import List, Optional

import numpy as np

STATE_UNRESTRICTED = 0xFFFFFFFE
STATE_INVALID = 0xFFFFFFFF
TABLE_BLOCK_ROWS = 4096


@dataclasses.dataclass
class Workload:
    name: str
    vocab: int
    hidden: int
    embedding: np.ndarray          # uint16 bits [V, H] (or float32 for cfg1)
    norm_weight: np.ndarray        # float32 [H]
    epsilon: float
    x: np.ndarray                  # float32 [B, H] (first step for cfg4)
    row_state: np.ndarray          # uint32 [B]
    state_offsets: np.ndarray      # uint32 [S + 1]
    state_tokens: np.ndarray       # uint32 [nnz]
    state_next: Optional[np.ndarray] = None   # uint32 [nnz] arcs
    next_table: Optional[np.ndarray] = None   # int32 [S, V] dense
    steps: int = 1
    seed: int = 0
    sizes: str = ""                # how the list sizes were drawn

    @property
    def rows(self) -> int:
        return int(self.x.shape[0])

    @property
    def states(self) -> int:
        return int(self.state_offsets.size - 1)

    @property
    def unrestricted_rows(self) -> np.ndarray:
        return np.nonzero(self.row_state == STATE_UNRESTRICTED)[0].astype(np.uint32)

    @property
    def max_count(self) -> int:
        d = np.diff(self.state_offsets.astype(np.int64))
        return int(d.max()) if d.size else 0

    def row_counts(self) -> np.ndarray:
        """Candidates per row (0 for unrestricted rows)."""
        out = np.zeros(self.rows, np.int64)
        rs = self.row_state.astype(np.int64)
        ok = rs < self.states
        off = self.state_offsets.astype(np.int64)
        out[ok] = off[rs[ok] + 1] - off[rs[ok]]
        return out

    def distinct_restricted_ids(self, rows: Optional[np.ndarray] = None) -> int:
        """U: distinct embedding rows touched by the restricted rows (or by the
        rows a boolean mask ``rows`` selects among them)."""
        seen = np.zeros(self.vocab, bool)
        off = self.state_offsets
        sel = self.row_state < self.states
        if rows is not None:
            sel = sel & rows
        for s in np.unique(self.row_state[sel]):
            seen[self.state_tokens[off[s]:off[s + 1]]] = True
        return int(seen.sum())

    def step_hidden(self, step: int) -> np.ndarray:
        """Hidden states of decode step ``step`` (cfg4 draws fresh N(0,1) per
        step from seed + step)."""
        if step == 0:
            return self.x
        rng = np.random.Generator(np.random.PCG64(
            np.random.SeedSequence([self.seed, 0x5EED, step])))
        return rng.standard_normal(self.x.shape, dtype=np.float32)


def _children(seed: int, n: int) -> List[np.random.Generator]:
    return [np.random.Generator(np.random.PCG64(s))
            for s in np.random.SeedSequence(seed).spawn(n)]


def normal_table_f16(rng: np.random.Generator, rows: int, cols: int,
                     scale: float) -> np.ndarray:
    """FP16 bits of scale * N(0,1), drawn in fixed row blocks."""
    out = np.empty((rows, cols), np.uint16)
    for r0 in range(0, rows, TABLE_BLOCK_ROWS):
        r1 = min(rows, r0 + TABLE_BLOCK_ROWS)
        block = rng.standard_normal((r1 - r0, cols), dtype=np.float32)
        block *= np.float32(scale)
        out[r0:r1] = block.astype(np.float16).view(np.uint16)
    return out


def normal_table_f32(rng, rows, cols, scale) -> np.ndarray:
    out = np.empty((rows, cols), np.float32)
    for r0 in range(0, rows, TABLE_BLOCK_ROWS):
        r1 = min(rows, r0 + TABLE_BLOCK_ROWS)
        block = rng.standard_normal((r1 - r0, cols), dtype=np.float32)
        block *= np.float32(scale)
        out[r0:r1] = block
    return out


def log_uniform_sizes(rng, n: int, hi: int) -> np.ndarray:
    """floor(exp(u * ln(hi + 1))), u ~ U[0, 1), clamped to [1, hi]."""
    u = rng.random(n)
    s = np.floor(np.exp(u * math.log(hi + 1.0))).astype(np.int64)
    return np.clip(s, 1, hi)


def distinct_sorted_ids(rng, vocab: int, k: int) -> np.ndarray:
    return np.sort(rng.choice(vocab, size=k, replace=False)).astype(np.uint32)


def lists_ascending(offsets: np.ndarray, tokens: np.ndarray) -> bool:
    """True when every CSR list tokens[offsets[s]:offsets[s + 1]] is strictly
    ascending (the layout MF_TAIL_SORTED_LISTS declares)."""
    t = np.asarray(tokens, dtype=np.int64)
    if t.size < 2:
        return True
    up = np.diff(t) > 0
    # pairs that straddle two lists are not compared
    ends = np.asarray(offsets, dtype=np.int64)[1:-1] - 1
    ends = ends[(ends >= 0) & (ends < up.size)]
    up[ends] = True
    return bool(up.all())


def _pack(lists: List[Optional[np.ndarray]]):
    """CSR over the restricted rows; None marks an unrestricted row."""
    offsets = [0]
    row_state = np.empty(len(lists), np.uint32)
    chunks = []
    s = 0
    for r, ids in enumerate(lists):
        if ids is None:
            row_state[r] = STATE_UNRESTRICTED
            continue
        chunks.append(ids)
        offsets.append(offsets[-1] + ids.size)
        row_state[r] = s
        s += 1
    tokens = np.concatenate(chunks) if chunks else np.zeros(0, np.uint32)
    return row_state, np.asarray(offsets, np.uint32), tokens.astype(np.uint32)


def ragged_pack(name: str, seed: int, vocab: int, hidden: int, rows: int,
                size_kind: str, size_hi: int, unrestricted_frac: float,
                size_lo: int = 1, emb_scale: float = 0.02) -> Workload:
    g_emb, g_x, g_w, g_size, g_ids, g_unr = _children(seed, 6)
    emb = normal_table_f16(g_emb, vocab, hidden, emb_scale)
    x = g_x.standard_normal((rows, hidden), dtype=np.float32)
    w = (np.float32(1.0) + np.float32(0.02) *
         g_w.standard_normal(hidden, dtype=np.float32)).astype(np.float32)
    if size_kind == "uniform":
        sizes = g_size.integers(size_lo, size_hi + 1, size=rows)
    else:
        sizes = log_uniform_sizes(g_size, rows, size_hi)
    sizes = np.minimum(sizes, vocab)
    n_unr = int(round(unrestricted_frac * rows))
    unr = set(g_unr.permutation(rows)[:n_unr].tolist())
    lists: List[Optional[np.ndarray]] = []
    for r in range(rows):
        if r in unr:
            lists.append(None)
        else:
            lists.append(distinct_sorted_ids(g_ids, vocab, int(sizes[r])))
    row_state, offsets, tokens = _pack(lists)
    return Workload(name=name, vocab=vocab, hidden=hidden, embedding=emb,
                    norm_weight=w, epsilon=1e-5, x=x, row_state=row_state,
                    state_offsets=offsets, state_tokens=tokens, seed=seed,
                    sizes=f"{'log-' if size_kind == 'log' else ''}uniform [{size_lo}, {size_hi}]")


def synthetic_dfa_tail(name: str, seed: int, vocab: int, hidden: int, rows: int,
                       states: int, lo: int, hi: int, steps: int) -> Workload:
    """cfg4: a token DFA with ``states`` states; each state's list has
    U[lo, hi] distinct random ids; dense next table int32 [S, V] with -1 off
    the list and a random next state on it; random start states."""
    g_emb, g_x, g_w, g_size, g_ids, g_next, g_start = _children(seed, 7)
    emb = normal_table_f16(g_emb, vocab, hidden, 0.02)
    x = g_x.standard_normal((rows, hidden), dtype=np.float32)
    w = (np.float32(1.0) + np.float32(0.02) *
         g_w.standard_normal(hidden, dtype=np.float32)).astype(np.float32)
    sizes = g_size.integers(lo, hi + 1, size=states)
    offsets = np.zeros(states + 1, np.uint32)
    chunks = []
    table = np.full((states, vocab), -1, np.int32)
    nexts = []
    for s in range(states):
        ids = distinct_sorted_ids(g_ids, vocab, int(sizes[s]))
        nxt = g_next.integers(0, states, size=ids.size).astype(np.uint32)
        table[s, ids] = nxt.astype(np.int32)
        chunks.append(ids)
        nexts.append(nxt)
        offsets[s + 1] = offsets[s] + ids.size
    start = g_start.integers(0, states, size=rows).astype(np.uint32)
    return Workload(name=name, vocab=vocab, hidden=hidden, embedding=emb,
                    norm_weight=w, epsilon=1e-5, x=x, row_state=start,
                    state_offsets=offsets,
                    state_tokens=np.concatenate(chunks).astype(np.uint32),
                    state_next=np.concatenate(nexts).astype(np.uint32),
                    next_table=table, steps=steps, seed=seed,
                    sizes=f"uniform [{lo}, {hi}] per DFA state")


def single_sequence_f32(seed: int = 0, vocab: int = 49152, hidden: int = 576,
                        allowed: int = 16) -> Workload:
    """cfg1: FP32 table N(0, 0.02), one N(0,1) hidden through the final
    RMSNorm (eps 1e-5, weight 1 + N(0, 0.02)), 16 distinct allowed ids."""
    g_emb, g_x, g_w, g_ids = _children(seed, 4)
    emb = normal_table_f32(g_emb, vocab, hidden, 0.02)
    x = g_x.standard_normal((1, hidden), dtype=np.float32)
    w = (np.float32(1.0) + np.float32(0.02) *
         g_w.standard_normal(hidden, dtype=np.float32)).astype(np.float32)
    ids = distinct_sorted_ids(g_ids, vocab, allowed)
    return Workload(name="cfg1", vocab=vocab, hidden=hidden, embedding=emb,
                    norm_weight=w, epsilon=1e-5, x=x,
                    row_state=np.zeros(1, np.uint32),
                    state_offsets=np.array([0, allowed], np.uint32),
                    state_tokens=ids, seed=seed)


def config(n: int, seed: int = 0, scale_vocab: Optional[int] = None,
           scale_rows: Optional[int] = None) -> Workload:
    """Benchmark configuration cfg<n>.  ``scale_vocab``/``scale_rows`` shrink a
    config for quick CPU checks (same generator, smaller shape)."""
    if n == 1:
        return single_sequence_f32(seed, vocab=scale_vocab or 49152)
    if n == 2:
        return ragged_pack("cfg2", seed, scale_vocab or 49152, 576,
                           scale_rows or 16, "uniform", 512, 0.0)
    if n == 3:
        return ragged_pack("cfg3", seed, scale_vocab or 49152, 576,
                           scale_rows or 256, "log", 4096, 0.10)
    if n == 4:
        return synthetic_dfa_tail("cfg4", seed, scale_vocab or 49152, 576,
                                  scale_rows or 64, 128, 2, 256, 32)
    if n == 5:
        return ragged_pack("cfg5", seed, scale_vocab or 128256, 2048,
                           scale_rows or 1024, "log", 16384, 0.05)
    raise ValueError(f"unknown config {n}")
