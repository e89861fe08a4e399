"""mf_decode_tail_f16_noalloc (the decode tail on the library's own per-GPU
workspace, no allocation) against mf_decode_tail_f16 with a caller workspace,
through the C ABI: two calls in a row, the second with a smaller pack, for
each kernel set the tail can take (table pass, gather + MFMA head, one-kernel
tail with whole lists and with lists in parts, dense head + gather), and each
against the oracle."""
import numpy as np
import pytest

import oracle
from market_sim_amd import abi, ops
from market_sim_amd import workloads as wl
from market_sim_amd.tail import DeviceTail

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _lib(hip):
    return hip


def _oracle(w):
    return oracle.decode_tail(w.x, w.norm_weight, w.epsilon, w.embedding, w.row_state,
                              w.state_offsets, w.state_tokens, state_next=w.state_next,
                              threads=8)


def _bits(out):
    tok, sc, nx = out
    return tok.copy(), sc.view(np.uint32).copy(), nx.copy()


def _same(a, b):
    for u, v in zip(a, b):
        assert np.array_equal(u, v)


def _noalloc(t):
    """The same arguments (the workspace field is not used) on the
    no-allocation entry point; the outputs land in the same buffers."""
    t.out_token.fill_(-7)
    t.out_score.fill_(-7.0)
    t.out_next.fill_(-7)
    import torch
    torch.cuda.synchronize()
    abi.check("noalloc", ops.decode_tail_f16_noalloc(t.args(), t.stream.cuda_stream))
    return _bits(t.results())


def _workloads(kind):
    if kind == "table_pass":
        big = wl.config(3, seed=51, scale_vocab=8192, scale_rows=200)
        small = wl.config(3, seed=52, scale_vocab=6000, scale_rows=48)
    elif kind == "gather":
        big = wl.config(3, seed=53, scale_vocab=8192, scale_rows=160)
        small = wl.config(2, seed=54, scale_vocab=5000, scale_rows=12)
    elif kind == "dense":  # wide rows, long ascending lists
        big = wl.ragged_pack("dense", 57, 5000, 1024, 64, "log", 4000, 0.05)
        small = wl.ragged_pack("dense", 58, 4000, 1024, 24, "log", 3000, 0.1)
    elif kind == "parts":  # one-kernel tail, lists in parts merged by the last part
        big = wl.ragged_pack("parts", 59, 6000, 576, 24, "uniform", 900, 0.0, size_lo=300)
        small = wl.ragged_pack("parts", 60, 3000, 576, 8, "uniform", 400, 0.0, size_lo=100)
    else:  # one-kernel tail: short lists, no unrestricted rows
        big = wl.synthetic_dfa_tail("short", 55, 8192, 576, 96, 32, 2, 100, 1)
        small = wl.synthetic_dfa_tail("short", 56, 4096, 576, 20, 16, 2, 60, 1)
    return big, small


@pytest.mark.parametrize("kind", ["table_pass", "gather", "fused", "parts", "dense"])
def test_noalloc_equals_workspace_entry_point_on_two_calls(kind):
    want_path = {"table_pass": abi.TAIL_PATH_TABLE_PASS, "gather": abi.TAIL_PATH_GATHER,
                 "fused": abi.TAIL_PATH_FUSED, "parts": abi.TAIL_PATH_FUSED,
                 "dense": abi.TAIL_PATH_DENSE}[kind]
    for w in _workloads(kind):
        # (the gather kind switches the one-kernel tail off: its small pack
        # would fit it)
        t = DeviceTail(w, sorted_lists=kind in ("table_pass", "dense"), fused=kind != "gather")
        assert ops.decode_tail_path(t.args()) == want_path
        assert ops.decode_tail_workspace_bytes(t.args()) <= ops.decode_tail_noalloc_max_bytes()
        ref = _bits(t.run())
        got = _noalloc(t)
        _same(got, ref)
        etok, esc, enx = _oracle(w)
        assert np.array_equal(got[0], etok)
        assert np.array_equal(got[2], enx)
        del t
