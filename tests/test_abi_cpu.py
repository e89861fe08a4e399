"""CPU checks of the C ABI: the library loads without a GPU, exports every
function the header declares, and rejects invalid metadata before any device
call (the reference's *_rejects_invalid_metadata tests, cuda_tests.cu)."""
import ctypes
import os
import re

import pytest

from market_sim_amd import abi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
FAKE_STREAM = 0x1000


def declared_functions():
    text = open(os.path.join(ROOT, "include", "marketforge_hip.h")).read()
    return sorted(set(re.findall(r"^\s*(?:mf_status|uint32_t|uint64_t)\s+(mf_\w+)\(", text, re.M)))


def test_header_declarations_match_binding():
    assert declared_functions() == sorted(abi.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = abi.lib()
    for name in declared_functions():
        assert hasattr(lib, name), name
    assert lib.mf_abi_version() == 6


def b(addr, n):
    return abi.Buffer(addr, n)


def test_greedy_rejects_invalid_metadata_before_launch():
    """cuda_tests.cu:1137-1167."""
    l = abi.lib()
    logits, tokens = b(0x10000, 16), b(0x20000, 4)
    assert l.mf_greedy_select_f16(logits, tokens, 0, 8, FAKE_STREAM).code == abi.MF_INVALID_ARGUMENT
    assert l.mf_greedy_select_f16(logits, tokens, 1, 8, 0).code == abi.MF_INVALID_ARGUMENT
    assert l.mf_greedy_select_f16(logits, tokens, 1, 7, FAKE_STREAM).code == abi.MF_INVALID_ARGUMENT
    assert l.mf_greedy_select_f16(logits, tokens, 1, 2 ** 32, FAKE_STREAM).code == abi.MF_RESOURCE_LIMIT
    assert l.mf_greedy_select_f16(logits, logits, 1, 8, FAKE_STREAM).code == abi.MF_INVALID_ARGUMENT


def test_restricted_greedy_rejects_invalid_metadata():
    """cuda_tests.cu:1256-1276."""
    l = abi.lib()
    logits, allowed, counts, out = b(0x10000, 16), b(0x20000, 16), b(0x30000, 4), b(0x40000, 4)
    f = l.mf_restricted_greedy_select_f16
    assert f(logits, allowed, counts, out, 1, 8, 0, FAKE_STREAM).code == abi.MF_INVALID_ARGUMENT
    assert f(logits, allowed, counts, out, 1, 8, 3, FAKE_STREAM).code == abi.MF_INVALID_ARGUMENT
    assert f(logits, allowed, counts, counts, 1, 8, 4, FAKE_STREAM).code == abi.MF_INVALID_ARGUMENT


def test_restricted_output_head_rejects_invalid_metadata():
    """cuda_tests.cu:1283-1339."""
    l = abi.lib()
    rows, hidden, vocab, mx = 1, 4, 8, 2
    h, e = b(0x10000, rows * hidden * 2), b(0x20000, vocab * hidden * 2)
    a, c, o = b(0x30000, rows * mx * 4), b(0x40000, rows * 4), b(0x50000, rows * 4)
    f = l.mf_restricted_output_head_f16
    assert f(h, e, a, c, o, 0, hidden, vocab, mx, FAKE_STREAM).code == abi.MF_INVALID_ARGUMENT
    assert f(h, e, a, c, o, rows, hidden, vocab, 0, FAKE_STREAM).code == abi.MF_INVALID_ARGUMENT
    assert f(h, e, a, c, o, rows, hidden, vocab, mx, 0).code == abi.MF_INVALID_ARGUMENT
    assert f(h, e, a, c, c, rows, hidden, vocab, mx, FAKE_STREAM).code == abi.MF_INVALID_ARGUMENT
    assert f(h, e, a, c, o, 2 ** 64 - 1, hidden, vocab, mx, FAKE_STREAM).code == abi.MF_RESOURCE_LIMIT


def test_rms_norm_rejects_invalid_metadata_before_launch():
    """cuda_tests.cu:914-945."""
    l = abi.lib()
    x, w, y = b(0x10000, 32), b(0x20000, 16), b(0x30000, 32)
    f = l.mf_rms_norm_f32
    assert f(x, w, y, 0, 4, 1e-5, FAKE_STREAM).code == abi.MF_INVALID_ARGUMENT
    assert f(x, w, y, 2, 4, float("nan"), FAKE_STREAM).code == abi.MF_INVALID_ARGUMENT
    assert f(x, w, y, 2, 4, 1e-5, 0).code == abi.MF_INVALID_ARGUMENT
    assert f(x, w, y, 1, 4, 1e-5, FAKE_STREAM).code == abi.MF_INVALID_ARGUMENT
    assert f(x, x, y, 2, 4, 1e-5, FAKE_STREAM).code == abi.MF_INVALID_ARGUMENT


def test_linear_rejects_invalid_metadata():
    l = abi.lib()
    f = l.mf_linear_f16
    x, w, y = b(0x10000, 12), b(0x20000, 12), b(0x30000, 8)
    assert f(x, w, y, 2, 3, 2, 0).code == abi.MF_INVALID_ARGUMENT
    assert f(x, w, y, 0, 3, 2, FAKE_STREAM).code == abi.MF_INVALID_ARGUMENT
    assert f(x, w, y, 2 ** 62, 3, 2, FAKE_STREAM).code == abi.MF_ARITHMETIC_OVERFLOW
    assert f(x, x, y, 2, 3, 2, FAKE_STREAM).code == abi.MF_INVALID_ARGUMENT


def test_copy_validation():
    """src/cuda/device_buffer.cu:15-33."""
    l = abi.lib()
    buf = b(0x10000, 16)
    host = ctypes.create_string_buffer(32)
    assert l.mf_copy_to_device_async(buf, 0, host, 8, 0).code == abi.MF_INVALID_ARGUMENT
    assert l.mf_copy_to_device_async(buf, 0, None, 8, FAKE_STREAM).code == abi.MF_INVALID_ARGUMENT
    assert l.mf_copy_to_device_async(buf, 12, host, 8, FAKE_STREAM).code == abi.MF_INVALID_ARGUMENT
    assert l.mf_copy_to_device_async(buf, 2 ** 64 - 4, host, 8, FAKE_STREAM).code == abi.MF_ARITHMETIC_OVERFLOW


def _tail_args(**over):
    rows, hidden, vocab, states, nnz = 4, 576, 1000, 4, 40
    a = abi.DecodeTailArgs()
    a.x = b(0x100000, rows * hidden * 4)
    a.norm_weight = b(0x200000, hidden * 4)
    a.epsilon = 1e-5
    a.order = 0
    a.embedding = b(0x300000, vocab * hidden * 2)
    a.row_state = b(0x400000, rows * 4)
    a.state_offsets = b(0x500000, (states + 1) * 4)
    a.state_tokens = b(0x600000, nnz * 4)
    a.out_token = b(0x700000, rows * 4)
    a.out_score = b(0x800000, rows * 4)
    a.workspace = b(0x900000, 1 << 24)
    a.rows, a.hidden, a.vocab, a.states, a.nnz, a.max_count = rows, hidden, vocab, states, nnz, 10
    for k, v in over.items():
        setattr(a, k, v)
    return a


def test_decode_tail_path_choice():
    """Which kernels run: the dense head (unrestricted stage) for ascending
    lists at hidden >= 1024 with hidden % 32 == 0, unless MF_TAIL_NO_DENSE;
    the CSR gather and the MFMA head otherwise."""
    l = abi.lib()
    path = ctypes.c_uint32()

    def path_of(flags, hidden, rows=1024, vocab=4096):
        a = _tail_args(flags=flags, rows=rows, hidden=hidden, vocab=vocab, max_count=min(4000, vocab),
                       x=b(0x10000000, rows * hidden * 4), norm_weight=b(0x20000000, hidden * 4),
                       embedding=b(0x30000000, vocab * hidden * 2),
                       row_state=b(0x40000000, rows * 4), out_token=b(0x50000000, rows * 4),
                       out_score=b(0x60000000, rows * 4), workspace=b(0x70000000, 1 << 30))
        assert l.mf_decode_tail_path(ctypes.byref(a), ctypes.byref(path)).code == abi.MF_OK
        return path.value

    assert path_of(abi.TAIL_SORTED_LISTS, 2048) == abi.TAIL_PATH_DENSE
    assert path_of(abi.TAIL_SORTED_LISTS, 1056) == abi.TAIL_PATH_DENSE
    assert path_of(abi.TAIL_SORTED_LISTS | abi.TAIL_NO_DENSE, 2048) == abi.TAIL_PATH_GATHER
    assert path_of(0, 2048) == abi.TAIL_PATH_GATHER
    # hidden below 1024 or not whole 32-feature steps
    assert path_of(abi.TAIL_SORTED_LISTS | abi.TAIL_NO_FUSED, 576) == abi.TAIL_PATH_GATHER
    assert path_of(abi.TAIL_SORTED_LISTS, 2040) == abi.TAIL_PATH_GATHER
    # more rows than the launch's panels hold (256 slots per 8 compute units)
    assert path_of(abi.TAIL_SORTED_LISTS, 1024, rows=9000, vocab=512) == abi.TAIL_PATH_GATHER


def test_decode_tail_validation():
    l = abi.lib()
    n = ctypes.c_uint64()
    a = _tail_args()
    assert l.mf_decode_tail_workspace_bytes(ctypes.byref(a), ctypes.byref(n)).code == abi.MF_OK
    assert n.value > 4 * 576 * 4
    assert l.mf_decode_tail_f16(ctypes.byref(a), 0).code == abi.MF_INVALID_ARGUMENT
    bad = _tail_args(rows=0)
    assert l.mf_decode_tail_f16(ctypes.byref(bad), FAKE_STREAM).code == abi.MF_INVALID_ARGUMENT
    bad = _tail_args(order=7)
    assert l.mf_decode_tail_f16(ctypes.byref(bad), FAKE_STREAM).code == abi.MF_INVALID_ARGUMENT
    bad = _tail_args(out_score=b(0x700000, 16))  # aliases out_token
    assert l.mf_decode_tail_f16(ctypes.byref(bad), FAKE_STREAM).code == abi.MF_INVALID_ARGUMENT
    bad = _tail_args(out_token=b(0x100000, 16))  # aliases x
    assert l.mf_decode_tail_f16(ctypes.byref(bad), FAKE_STREAM).code == abi.MF_INVALID_ARGUMENT
    bad = _tail_args(x=b(0x100000, 12))  # wrong size
    assert l.mf_decode_tail_f16(ctypes.byref(bad), FAKE_STREAM).code == abi.MF_INVALID_ARGUMENT
    bad = _tail_args(workspace=b(0x900000, 64))  # too small
    assert l.mf_decode_tail_f16(ctypes.byref(bad), FAKE_STREAM).code == abi.MF_INVALID_ARGUMENT
    bad = _tail_args(max_count=5000)  # longer than the vocabulary
    assert l.mf_decode_tail_f16(ctypes.byref(bad), FAKE_STREAM).code == abi.MF_RESOURCE_LIMIT
    bad = _tail_args(unrestricted_count=2)  # rows list missing
    assert l.mf_decode_tail_f16(ctypes.byref(bad), FAKE_STREAM).code == abi.MF_INVALID_ARGUMENT


def test_decode_tail_sequence_table_and_flags_validation():
    """The sequence table: row_sequence sized by rows, a state table of any
    whole-entry size, next states of the table's size that may update it in
    place; unknown flag bits are rejected."""
    l = abi.lib()
    n = ctypes.c_uint64()
    rs = _tail_args().row_state

    def ws_code(**kw):
        a = _tail_args(**kw)
        return l.mf_decode_tail_workspace_bytes(ctypes.byref(a), ctypes.byref(n)).code

    table = b(rs.address, 40)                       # 10 entries for 4 rows
    seq = b(0xA00000, 16)
    assert ws_code(row_state=table, row_sequence=seq) == abi.MF_OK
    assert ws_code(row_state=table, row_sequence=seq, out_next_state=table) == abi.MF_OK
    assert ws_code(row_state=table, row_sequence=seq, out_next_state=b(0xB00000, 40)) == abi.MF_OK
    assert ws_code(row_state=table, row_sequence=seq,
                   out_next_state=b(0xB00000, 16)) == abi.MF_INVALID_ARGUMENT
    assert ws_code(row_state=table, row_sequence=b(0xA00000, 12)) == abi.MF_INVALID_ARGUMENT
    assert ws_code(row_state=b(rs.address, 42), row_sequence=seq) == abi.MF_INVALID_ARGUMENT
    assert ws_code(row_state=table) == abi.MF_INVALID_ARGUMENT   # no table: rows entries
    # without a sequence table the next states must not overwrite the states
    assert ws_code(out_next_state=rs) == abi.MF_INVALID_ARGUMENT
    assert ws_code(row_state=table, row_sequence=seq, out_token=seq) == abi.MF_INVALID_ARGUMENT
    assert ws_code(flags=abi.TAIL_HOLD_FINISHED) == abi.MF_OK
    assert ws_code(flags=abi.TAIL_SORTED_LISTS) == abi.MF_OK
    assert ws_code(flags=abi.TAIL_HOLD_FINISHED | abi.TAIL_SORTED_LISTS) == abi.MF_OK
    assert ws_code(flags=abi.TAIL_SORTED_LISTS | abi.TAIL_TABLE_PASS) == abi.MF_OK
    assert ws_code(flags=abi.TAIL_NO_FUSED) == abi.MF_OK
    assert ws_code(flags=abi.TAIL_SORTED_LISTS | abi.TAIL_NO_DENSE) == abi.MF_OK
    assert ws_code(flags=32) == abi.MF_INVALID_ARGUMENT


def test_sorted_lists_flag_sizes_the_range_index():
    """MF_TAIL_SORTED_LISTS adds the table pass's range index to the
    workspace where the pass runs (unrestricted rows or MF_TAIL_TABLE_PASS,
    hidden % 64 == 0, hidden <= 576, rows <= 256) and changes nothing where
    it does not."""
    l = abi.lib()
    n = ctypes.c_uint64()

    def ws(**kw):
        a = _tail_args(**kw)
        assert l.mf_decode_tail_workspace_bytes(ctypes.byref(a), ctypes.byref(n)).code == abi.MF_OK
        return n.value

    sorted_pass = abi.TAIL_SORTED_LISTS | abi.TAIL_TABLE_PASS
    assert ws(flags=sorted_pass) > ws()
    path = ctypes.c_uint32()

    def path_of(**kw):
        a = _tail_args(**kw)
        assert l.mf_decode_tail_path(ctypes.byref(a), ctypes.byref(path)).code == abi.MF_OK
        return path.value

    nf = abi.TAIL_NO_FUSED
    assert path_of(flags=sorted_pass) == abi.TAIL_PATH_TABLE_PASS
    assert path_of(flags=sorted_pass | nf) == abi.TAIL_PATH_TABLE_PASS
    assert path_of(flags=abi.TAIL_SORTED_LISTS | nf) == abi.TAIL_PATH_GATHER
    assert path_of(flags=nf) == abi.TAIL_PATH_GATHER
    assert path_of(flags=abi.TAIL_TABLE_PASS | nf) == abi.TAIL_PATH_GATHER
    # short lists and no unrestricted rows: the one-kernel tail
    assert path_of() == abi.TAIL_PATH_FUSED
    assert path_of(flags=abi.TAIL_SORTED_LISTS) == abi.TAIL_PATH_FUSED
    assert path_of(max_count=128) == abi.TAIL_PATH_FUSED
    # longer lists in parts of a workgroup's stage (128 candidate rows at
    # hidden 576), up to 16 parts, while the pack fits two workgroups per
    # compute unit (256 CUs)
    assert path_of(max_count=129) == abi.TAIL_PATH_FUSED

    def many(rows, max_count, vocab=4096):
        return dict(rows=rows, max_count=max_count, vocab=vocab,
                    x=b(0x10000000, rows * 576 * 4), embedding=b(0x30000000, vocab * 576 * 2),
                    row_state=b(0x40000000, rows * 4), out_token=b(0x50000000, rows * 4),
                    out_score=b(0x60000000, rows * 4), workspace=b(0x70000000, 1 << 30))

    assert path_of(**many(256, 256)) == abi.TAIL_PATH_FUSED      # 512 workgroups
    assert path_of(**many(257, 256)) == abi.TAIL_PATH_GATHER
    assert path_of(**many(16, 2048)) == abi.TAIL_PATH_FUSED      # 16 parts
    assert path_of(**many(16, 2049)) == abi.TAIL_PATH_GATHER
    assert path_of(flags=nf, **many(16, 512)) == abi.TAIL_PATH_GATHER
    unr = dict(unrestricted_count=1, unrestricted_rows=b(0xC00000, 4))
    assert path_of(flags=abi.TAIL_SORTED_LISTS, **unr) == abi.TAIL_PATH_TABLE_PASS
    assert path_of(**unr) == abi.TAIL_PATH_GATHER
    # without unrestricted rows the pass runs only when asked for
    assert ws(flags=abi.TAIL_SORTED_LISTS) == ws()
    wide = dict(hidden=2048, x=b(0x100000, 4 * 2048 * 4), norm_weight=b(0x200000, 2048 * 4),
                embedding=b(0x300000, 1000 * 2048 * 2))
    assert ws(flags=sorted_pass, **wide) == ws(**wide)


def test_decode_tail_noalloc_rejects_before_any_device_call():
    """mf_decode_tail_f16_noalloc: validation as for mf_decode_tail_f16, and
    a call whose workspace exceeds the library's per-GPU array is a resource
    limit, reported before anything touches a device."""
    l = abi.lib()
    assert l.mf_decode_tail_noalloc_max_bytes() == 16 << 20
    a = _tail_args()
    assert l.mf_decode_tail_f16_noalloc(ctypes.byref(a), 0).code == abi.MF_INVALID_ARGUMENT
    assert l.mf_decode_tail_f16_noalloc(None, FAKE_STREAM).code == abi.MF_INVALID_ARGUMENT
    bad = _tail_args(rows=0)
    assert l.mf_decode_tail_f16_noalloc(ctypes.byref(bad), FAKE_STREAM).code == \
        abi.MF_INVALID_ARGUMENT
    # 1024 rows of a 2048-wide hidden with lists up to 16384 ids: a 45 MB workspace
    rows, hidden, vocab, states, nnz = 1024, 2048, 128256, 1024, 1 << 20
    big = _tail_args(rows=rows, hidden=hidden, vocab=vocab, states=states, nnz=nnz,
                     max_count=16384)
    big.x = b(0x10000000, rows * hidden * 4)
    big.norm_weight = b(0x20000000, hidden * 4)
    big.embedding = b(0x30000000, vocab * hidden * 2)
    big.row_state = b(0x40000000, rows * 4)
    big.state_offsets = b(0x50000000, (states + 1) * 4)
    big.state_tokens = b(0x60000000, nnz * 4)
    big.out_token = b(0x70000000, rows * 4)
    big.out_score = b(0x80000000, rows * 4)
    n = ctypes.c_uint64()
    assert l.mf_decode_tail_workspace_bytes(ctypes.byref(big), ctypes.byref(n)).code == abi.MF_OK
    assert n.value > l.mf_decode_tail_noalloc_max_bytes()
    assert l.mf_decode_tail_f16_noalloc(ctypes.byref(big), FAKE_STREAM).code == \
        abi.MF_RESOURCE_LIMIT
