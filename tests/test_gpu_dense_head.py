"""GPU parity of the dense head (mf_dense.hip): the unrestricted rows and the
long ascending lists scored by one MFMA pass over the table, selected
against the CPU oracle bit for bit (tokens, scores, next states), and equal
to the gather path (MF_TAIL_NO_DENSE) on the same inputs.

The dense head runs for ascending lists at hidden >= 1024 (hidden % 32 ==
0); among the lists of at least max(64, vocab / 256) ids the device takes
the longest: as many as fill the room the unrestricted rows leave in their
panels of 256 slots, then whole panels while a panel's lists hold at least
5/2 vocab ids.
"""
import numpy as np
import pytest

import oracle
from market_sim_amd import abi
from market_sim_amd import workloads as wl

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _lib(hip):
    return hip


def _oracle(w, x=None, order=abi.ORDER_FMA_CHAIN, threads=16):
    return oracle.decode_tail(w.x if x is None else x, w.norm_weight, w.epsilon,
                              w.embedding, w.row_state, w.state_offsets, w.state_tokens,
                              state_next=w.state_next, next_table=w.next_table, order=order,
                              threads=threads)


def _tail(w, **kw):
    """The decode tail without the one-kernel tail (MF_TAIL_NO_FUSED), which
    takes small packs without unrestricted rows before the dense head is
    considered; these tests are about the dense head and the gather."""
    from market_sim_amd.tail import DeviceTail
    kw.setdefault("sorted_lists", True)
    kw.setdefault("fused", False)
    return DeviceTail(w, **kw)


def _bits(a):
    return np.asarray(a).view(np.uint32)


def _same(got, exp):
    tok, sc, nx = got
    etok, esc, enx = exp
    bad = np.nonzero(tok != etok)[0]
    assert bad.size == 0, f"token mismatch rows {bad[:10]}: got {tok[bad[:10]]} want {etok[bad[:10]]}"
    nan = np.isnan(esc)
    assert np.array_equal(np.isnan(sc), nan)
    diff = np.nonzero((_bits(sc) != _bits(esc)) & ~nan)[0]
    assert diff.size == 0, f"score bits differ in rows {diff[:8]}"
    assert np.array_equal(nx, enx)


def _dense_and_gather(w, exp=None, **kw):
    """The dense head's result, the gather's, and the oracle's all agree."""
    t = _tail(w, **kw)
    assert t.dense
    got = t.run()
    g = _tail(w, dense=False, **kw)
    assert not g.dense
    gathered = g.run()
    for a, b in zip(got, gathered):
        assert np.array_equal(_bits(a), _bits(b))
    _same(got, _oracle(w) if exp is None else exp)
    return got


def _pack(seed, vocab, hidden, rows, longest, unrestricted, size_kind="log", size_lo=1):
    return wl.ragged_pack("dense", seed, vocab, hidden, rows, size_kind, longest, unrestricted,
                          size_lo=size_lo)


def test_scaled_cfg5_with_unrestricted_rows():
    """configs[4]'s shape family (H = 2048, 5% unrestricted) on a 20000-token
    vocabulary: the last tile is partial (20000 = 104 x 192 + 32)."""
    w = wl.config(5, seed=2, scale_vocab=20000, scale_rows=96)
    assert w.unrestricted_rows.size > 0
    _dense_and_gather(w)


def test_no_unrestricted_rows_long_lists():
    """No unrestricted rows: the long lists hold more than 5/2 vocab ids, so
    the dense head takes them; a 1056-wide hidden row (33 MFMA steps)."""
    w = _pack(3, 12000, 1056, 64, 8192, 0.0)
    lens = np.diff(w.state_offsets.astype(np.int64))[w.row_state]
    assert lens[lens >= 64].sum() >= 5 * w.vocab // 2
    _dense_and_gather(w)


def test_few_long_lists_stay_on_the_gather():
    """Lists long enough for the dense head but too few ids in all (and no
    unrestricted rows): the device keeps them on the gather; exact either
    way."""
    w = _pack(4, 12000, 1024, 6, 1500, 0.0)
    lens = np.diff(w.state_offsets.astype(np.int64))[w.row_state]
    assert lens.max() >= 64 and lens.sum() < 5 * w.vocab // 2
    _dense_and_gather(w)


def test_lists_not_ascending_are_left_to_the_gather():
    """MF_TAIL_SORTED_LISTS declared for lists that are not ascending (two
    long lists shuffled, one with a repeated id): the norm launch's walk
    rejects them and the gather scores them; results stay exact."""
    w = _pack(5, 9000, 1024, 48, 6000, 0.05)
    offs = w.state_offsets.astype(np.int64)
    lens = np.diff(offs)
    tokens = w.state_tokens.copy()
    rng = np.random.default_rng(0)
    long_states = [s for s in np.unique(w.row_state[w.row_state < w.states]) if lens[s] >= 200]
    assert len(long_states) >= 2
    s0, s1 = long_states[:2]
    seg = tokens[offs[s0]:offs[s0 + 1]]
    rng.shuffle(seg)
    tokens[offs[s0]:offs[s0 + 1]] = seg
    tokens[offs[s1] + 7] = tokens[offs[s1] + 6]
    w.state_tokens = tokens
    _dense_and_gather(w, sorted_lists=True)


def test_bad_id_nan_hidden_and_exact_ties():
    """A long list holding an id >= V (the row is invalid), a row whose
    hidden vector is NaN (its lowest id, greedy.cu's all-NaN rule), and rows
    whose whole list shares one embedding row (the lowest id wins)."""
    w = _pack(6, 8000, 1024, 40, 4000, 0.05)
    w.x = w.x.copy()
    w.embedding = w.embedding.copy()
    offs = w.state_offsets.astype(np.int64)
    lens = np.diff(offs)
    rows = [r for r in range(w.rows) if w.row_state[r] < w.states and lens[w.row_state[r]] >= 100]
    assert len(rows) >= 4
    tokens = w.state_tokens.copy()
    # the last id of the first row's list past the vocabulary (still ascending)
    s_bad = int(w.row_state[rows[0]])
    tokens[offs[s_bad + 1] - 1] = w.vocab + 9
    w.state_tokens = tokens
    w.x[rows[1]] = np.nan
    tied = []
    used = set()
    for r in rows[2:]:
        s = int(w.row_state[r])
        ids = w.state_tokens[offs[s]:offs[s + 1]]
        if not (set(ids.tolist()) & used):
            w.embedding[ids] = w.embedding[ids[len(ids) // 2]]
            used |= set(ids.tolist())
            tied.append((r, int(ids.min())))
        if len(tied) == 2:
            break
    assert tied
    got = _dense_and_gather(w)
    assert got[0][rows[0]] == abi.INVALID_TOKEN
    s1 = int(w.row_state[rows[1]])
    assert got[0][rows[1]] == w.state_tokens[offs[s1]:offs[s1 + 1]].min()
    for r, lowest in tied:
        assert got[0][r] == lowest


@pytest.mark.parametrize("order", [abi.ORDER_FMA_CHAIN, abi.ORDER_MUL_ADD_CHAIN])
def test_extreme_row_scales_and_near_ties(order):
    """Rows scaled from 1e-20 to 1e18, and near-tied candidates (an embedding
    row and a copy one FP16 ulp apart in one feature) in long lists."""
    w = _pack(7, 9000, 1024, 50, 5000, 0.06)
    w.embedding = w.embedding.copy()
    rng = np.random.default_rng(3)
    offs = w.state_offsets.astype(np.int64)
    for r in range(w.rows):
        s = int(w.row_state[r])
        if s >= w.states or offs[s + 1] - offs[s] < 2:
            continue
        a, b = int(w.state_tokens[offs[s]]), int(w.state_tokens[offs[s] + 1])
        w.embedding[b] = w.embedding[a]
        f = int(rng.integers(0, w.hidden))
        w.embedding[b, f] = w.embedding[b, f] + 1
    scales = np.array([1e-20, 1e-6, 1.0, 1e6, 1e18], np.float32)
    w.x = (w.x * scales[np.arange(w.rows) % scales.size][:, None]).astype(np.float32)
    t = _tail(w, order=order)
    assert t.dense
    _same(t.run(), _oracle(w, order=order))


def test_duplicate_and_foreign_unrestricted_rows():
    """The unrestricted list names a row twice and a restricted row with a
    long list (which the dense head also takes as a list row)."""
    w = _pack(8, 7000, 1024, 40, 5000, 0.1)
    lens = np.diff(w.state_offsets.astype(np.int64))
    restricted = [r for r in range(w.rows) if w.row_state[r] < w.states and lens[w.row_state[r]] >= 64]
    unr = w.unrestricted_rows
    listed = np.concatenate([unr, unr[:1], np.array(restricted[:1])]).astype(np.uint32)
    t = _tail(w, unrestricted=listed)
    assert t.dense
    _same(t.run(), _oracle(w))


def test_repeated_calls_and_stages():
    """Repeated calls on one workspace give the same bits, and so do the four
    stage entry points called one by one."""
    from market_sim_amd import ops
    w = _pack(9, 10000, 1024, 72, 8192, 0.05)
    t = _tail(w)
    first = t.run()
    for _ in range(4):
        again = t.run()
        for a, b in zip(first, again):
            assert np.array_equal(_bits(a), _bits(b))
    a = t.args()
    h = t.stream.cuda_stream
    for fn in (ops.decode_tail_prepare, ops.decode_tail_restricted,
               ops.decode_tail_unrestricted, ops.decode_tail_finalize):
        abi.check("stage", fn(a, h))
    staged = t.results()
    for x, y in zip(first, staged):
        assert np.array_equal(_bits(x), _bits(y))
    _same(first, _oracle(w))


def test_unrestricted_rows_fill_two_panels():
    """More than 256 unrestricted rows (300 of 600): the dense head runs
    P >= 2 panels of equal size, so the slot split across panels, the
    per-XCD groups of P workgroups and fb_map written by every panel's first
    group are exercised; exact against the oracle and the gather."""
    w = _pack(12, 6000, 1024, 600, 4096, 0.5)
    assert w.unrestricted_rows.size > 256
    _dense_and_gather(w)


def test_long_lists_take_a_second_panel():
    """No unrestricted rows and 300 long ascending lists (2000-4000 ids of a
    6000-token vocabulary): the device fills the first panel with the 256
    longest and, since the remaining 44 lists still hold more than 5/2 vocab
    ids, takes them as a second panel (slots > 256); exact against the
    oracle and the gather."""
    w = _pack(13, 6000, 1024, 300, 4000, 0.0, size_kind="uniform", size_lo=2000)
    lens = np.sort(np.diff(w.state_offsets.astype(np.int64))[w.row_state])[::-1]
    dense_min = max(64, w.vocab // 256)
    assert (lens >= dense_min).sum() == 300
    assert lens[256:].sum() >= 5 * w.vocab // 2
    _dense_and_gather(w)


def test_more_candidate_lists_than_the_ranking_threads():
    """1100 ascending lists of 300-600 ids, every one long enough for the
    dense head: more candidates than the row choice ranks by counting
    (1024), so it sorts them (bitonic); the longest fill whole panels while
    a panel's lists hold 5/2 vocab ids (five panels here); exact against the
    oracle and the gather."""
    w = _pack(14, 6000, 1024, 1100, 600, 0.0, size_kind="uniform", size_lo=300)
    lens = np.diff(w.state_offsets.astype(np.int64))[w.row_state]
    assert (lens >= max(64, w.vocab // 256)).sum() > 1024
    _dense_and_gather(w)


def test_decode_steps_with_device_states():
    """A DFA tail at hidden 1024 with long lists: states carried on the device
    from step to step, every step exact."""
    rng = np.random.default_rng(11)
    vocab, hidden, rows, states = 6000, 1024, 32, 24
    offs = [0]
    toks = []
    for s in range(states):
        n = int(rng.integers(30, 2500))
        toks.append(np.sort(rng.choice(vocab, n, replace=False)).astype(np.uint32))
        offs.append(offs[-1] + n)
    tokens = np.concatenate(toks)
    nxt = rng.integers(0, states, tokens.size).astype(np.uint32)
    emb = (rng.standard_normal((vocab, hidden)) * 0.02).astype(np.float16).view(np.uint16)
    w = wl.Workload(name="dfa1024", vocab=vocab, hidden=hidden, embedding=emb,
                    norm_weight=(1 + 0.02 * rng.standard_normal(hidden)).astype(np.float32),
                    epsilon=1e-5, x=rng.standard_normal((rows, hidden)).astype(np.float32),
                    row_state=rng.integers(0, states, rows).astype(np.uint32),
                    state_offsets=np.array(offs, np.uint32), state_tokens=tokens, state_next=nxt)
    t = _tail(w)
    assert t.dense
    state = w.row_state.copy()
    for step in range(4):
        x = rng.standard_normal((rows, hidden)).astype(np.float32)
        t.set_hidden(x)
        got = t.run()
        exp = _oracle(wl.Workload(**{**w.__dict__, "row_state": state}), x=x)
        _same(got, exp)
        t.set_state(t.out_next)
        state = exp[2]
