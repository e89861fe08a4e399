"""The one-kernel decode tail (packs of short lists, no unrestricted rows)
against the CPU oracle and against the separate kernels (MF_TAIL_NO_FUSED),
bit for bit: tokens, scores and next states.

The packs hold lists of up to 128 ids (the one-kernel tail's limit).  At
H = 576 every list fits one workgroup stage of candidate rows; at H = 1024
the stage holds 71 rows, so longer lists take a second round.
The edge cases follow the reference's selection rules (greedy.cu:84-100,
163-166, 177-211): ids outside the vocabulary make the row invalid, an
all-NaN row takes its lowest id, equal scores go to the lowest id."""
import numpy as np
import pytest

import oracle
from market_sim_amd import abi
from market_sim_amd import workloads as wl

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _lib(hip):
    return hip


def _pack(seed, rows=64, vocab=6000, size_hi=128, hidden=576, size_lo=1):
    return wl.ragged_pack("short", seed, vocab, hidden, rows, "uniform", size_hi, 0.0,
                          size_lo=size_lo)


def _stage_rows(hidden):
    """Candidate rows one workgroup stages per round (156 KiB of LDS for x,
    the weight, the squares and rows of hidden + 8 halves)."""
    return min((156 * 1024 - 12 * hidden) // (2 * hidden + 16), 128)


def _oracle(w, order=abi.ORDER_FMA_CHAIN):
    return oracle.decode_tail(w.x, w.norm_weight, w.epsilon, w.embedding, w.row_state,
                              w.state_offsets, w.state_tokens, state_next=w.state_next,
                              next_table=w.next_table, order=order, threads=8)


def _bits_equal(got, exp):
    tok, sc, nx = got
    etok, esc, enx = exp
    bad = np.nonzero(tok != etok)[0]
    assert bad.size == 0, f"token mismatch rows {bad[:10]}: got {tok[bad[:10]]} want {etok[bad[:10]]}"
    nan = np.isnan(esc)
    assert np.array_equal(np.isnan(sc), nan)
    diff = np.nonzero((sc.view(np.uint32) != esc.view(np.uint32)) & ~nan)[0]
    assert diff.size == 0, f"score bits differ in rows {diff[:8]}"
    assert np.array_equal(nx, enx)


def _both(w, order=abi.ORDER_FMA_CHAIN):
    """(fused results, separate-kernel results); checks the fused path ran."""
    from market_sim_amd.tail import DeviceTail
    fused = DeviceTail(w, order=order)
    assert fused.fused, "the pack should take the one-kernel tail"
    sep = DeviceTail(w, order=order, fused=False)
    assert not sep.fused
    return fused.run(), sep.run()


@pytest.mark.parametrize("hidden", [576, 1024])
@pytest.mark.parametrize("order", [abi.ORDER_FMA_CHAIN, abi.ORDER_MUL_ADD_CHAIN])
def test_fused_tail_matches_oracle_and_separate_kernels(order, hidden):
    w = _pack(41, hidden=hidden)
    counts = np.diff(w.state_offsets.astype(np.int64))[w.row_state]
    if hidden == 1024:
        assert counts.max() > _stage_rows(hidden), "some row needs a second round of the stage"
    got, sep = _both(w, order)
    _bits_equal(got, _oracle(w, order))
    _bits_equal(got, sep)


def test_fused_tail_invalid_rows_bad_ids_nan_and_empty_lists():
    w = _pack(42, rows=32, hidden=1024)
    w.row_state = w.row_state.copy()
    w.x = w.x.copy()
    w.state_tokens = w.state_tokens.copy()
    # state beyond the table -> invalid row
    w.row_state[0] = w.states + 5
    # an out-of-vocabulary id in one list (first and, in another row, last
    # position of a two-round list) -> that row invalid
    w.state_tokens[w.state_offsets[w.row_state[1]]] = w.vocab + 3
    counts = np.diff(w.state_offsets.astype(np.int64))
    long_rows = [r for r in range(4, w.rows) if counts[w.row_state[r]] > _stage_rows(1024)]
    assert long_rows
    r_long = long_rows[0]
    w.state_tokens[w.state_offsets[w.row_state[r_long] + 1] - 1] = w.vocab
    # all-NaN hidden -> the lowest id of the list, with its own (NaN) score
    w.x[2] = np.nan
    # an empty list
    offs = w.state_offsets.astype(np.int64)
    s3 = int(w.row_state[3])
    new_tokens = np.concatenate([w.state_tokens[:offs[s3]], w.state_tokens[offs[s3 + 1]:]])
    offs[s3 + 1:] -= offs[s3 + 1] - offs[s3]
    w.state_tokens = new_tokens.astype(np.uint32)
    w.state_offsets = offs.astype(np.uint32)
    got, sep = _both(w)
    _bits_equal(got, _oracle(w))
    _bits_equal(got, sep)
    for r in (0, 1, 3, r_long):
        assert got[0][r] == abi.INVALID_TOKEN
    lo = w.state_tokens[w.state_offsets[w.row_state[2]]:w.state_offsets[w.row_state[2] + 1]].min()
    assert got[0][2] == lo and np.isnan(got[1][2])


def test_fused_tail_exact_ties_pick_the_lowest_id():
    """A whole list sharing one embedding row gives bit-identical scores;
    the lowest id wins, also when the tie spans both rounds of the stage."""
    w = _pack(43, rows=24, hidden=1024)
    w.embedding = w.embedding.copy()
    tied, used = [], set()
    sizes = np.diff(w.state_offsets.astype(np.int64))[w.row_state]
    for r in np.argsort(-sizes, kind="stable"):
        s = int(w.row_state[r])
        ids = w.state_tokens[w.state_offsets[s]:w.state_offsets[s + 1]]
        if ids.size >= 2 and not (set(ids.tolist()) & used):
            w.embedding[ids] = w.embedding[ids[-1]]
            used |= set(ids.tolist())
            tied.append((r, ids.min(), ids.size))
    assert any(n > _stage_rows(1024) for _, _, n in tied)
    got, sep = _both(w)
    _bits_equal(got, _oracle(w))
    _bits_equal(got, sep)
    for r, lowest, _ in tied:
        assert got[0][r] == lowest


def test_fused_tail_without_norm_weight():
    """norm_weight absent: x is taken as already normalized."""
    w = _pack(44, rows=48)
    w.norm_weight = None
    got, sep = _both(w)
    _bits_equal(got, _oracle(w))
    _bits_equal(got, sep)


def test_fused_tail_one_row_and_max_lists():
    """B = 1, and a pack whose every list has the full 128 ids."""
    w = _pack(45, rows=1)
    got, sep = _both(w)
    _bits_equal(got, _oracle(w))
    w = _pack(46, rows=16, size_lo=128)
    got, sep = _both(w)
    _bits_equal(got, _oracle(w))
    _bits_equal(got, sep)
