"""CPU oracle for the restricted output head (TEST INFRASTRUCTURE ONLY).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this package, and only as the checker: the
product path (``market_sim_amd``) never calls it and has no CPU fallback.

``liboracle.so`` (``oracle/oracle.c``) restates the reference's FP32 CPU loops
in their operation order; ``_ref/libmfref.so`` is the reference's own CPU code
compiled in place (present only where the reference tree was available at
build time) and is used to pin the restatement.

Pinning status per function (tests that pin it):
  half<->float          exhaustive vs numpy float16 (test_oracle_golden.py)
  rms_norm_f32          bit-exact vs reference operators.cpp (_ref) + hand values
  rms_norm_f16          numpy RNE half of the reference rms_norm_f32 (_ref),
                        subnormal and overflowing outputs included
  dot_fma               exact rational chain; tiny-head known answer
  dot_mul_add           bit-exact vs reference linear_f32 (_ref) + [-2, 3]
  FP32-table dots       exact rational chains in both orders (cfg1 path)
  selection rules       reference test cases (ties, NaN, sentinels), real logits
  decode_tail           float64 brute force + margin, one-hot closed forms,
                        real market DFA advance vs reference TokenDfa (_ref)
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
INVALID_TOKEN = 0xFFFFFFFF
STATE_UNRESTRICTED = 0xFFFFFFFE
ORDER_FMA_CHAIN = 0
ORDER_MUL_ADD_CHAIN = 1

_lib: Optional[ctypes.CDLL] = None
_ref: Optional[ctypes.CDLL] = None

_P = ctypes.c_void_p
_U64 = ctypes.c_uint64
_F = ctypes.c_float
_I = ctypes.c_int


def build() -> None:
    """Compile liboracle.so and, when the reference tree exists, _ref."""
    import subprocess

    subprocess.run(["make", "-s", "-C", HERE, "all"], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        path = os.path.join(HERE, "liboracle.so")
        if not os.path.exists(path):
            build()
        l = ctypes.CDLL(path)
        l.orc_half_to_float.restype = _F
        l.orc_half_to_float.argtypes = [ctypes.c_uint16]
        l.orc_float_to_half.restype = ctypes.c_uint16
        l.orc_float_to_half.argtypes = [_F]
        l.orc_half_to_float_n.argtypes = [_P, _P, _U64]
        l.orc_rms_norm_f32.argtypes = [_P, _P, _F, _P, _U64, _U64]
        l.orc_rms_norm_f16.argtypes = [_P, _P, _F, _P, _U64, _U64]
        l.orc_dot_fma.restype = _F
        l.orc_dot_fma.argtypes = [_P, _P, _U64]
        l.orc_dot_mul_add.restype = _F
        l.orc_dot_mul_add.argtypes = [_P, _P, _U64]
        l.orc_greedy_f16.argtypes = [_P, _U64, _U64, _P]
        l.orc_restricted_greedy_f16.argtypes = [_P, _P, _P, _U64, _U64, _U64, _P]
        l.orc_greedy_f32.argtypes = [_P, _U64, _U64, _P]
        l.orc_restricted_greedy_f32.argtypes = [_P, _P, _P, _U64, _U64, _U64, _P]
        l.orc_restricted_output_head_f16.argtypes = [
            _P, _P, _P, _P, _U64, _U64, _U64, _U64, _P, _P]
        l.orc_linear_f16.argtypes = [_P, _P, _U64, _U64, _U64, _P, _P]
        l.orc_decode_tail.restype = _I
        l.orc_decode_tail.argtypes = [
            _P, _P, _F, _P, _P, _U64, _U64, _P, _U64, _P, _P, _U64, _P, _P, _I,
            _P, _P, _P, _I]
        l.orc_scores.argtypes = [_P, _P, _U64, _P, _U64, _I, _P]
        _lib = l
    return _lib


def ref() -> Optional[ctypes.CDLL]:
    """The reference's own CPU code (oracle/_ref), or None if not built."""
    global _ref
    if _ref is None:
        path = os.path.join(HERE, "_ref", "libmfref.so")
        if not os.path.exists(path):
            return None
        r = ctypes.CDLL(path)
        r.mfref_rms_norm_f32.restype = _I
        r.mfref_rms_norm_f32.argtypes = [_P, _P, _F, _P, _U64, _U64]
        r.mfref_linear_f32.restype = _I
        r.mfref_linear_f32.argtypes = [_P, _P, _P, _U64, _U64, _U64]
        u32 = ctypes.c_uint32
        r.mfref_token_dfa_export.restype = _I
        r.mfref_token_dfa_export.argtypes = [
            _P, _P, _P, u32, u32, u32, u32, u32, u32, _P, _P, _P, _P, u32, u32,
            _P, _P]
        r.mfref_token_dfa_advance.restype = _I
        r.mfref_token_dfa_advance.argtypes = [_P, _P, _P, u32, u32, u32, u32, _P]
        r.mfref_market_dfa_export.restype = _I
        r.mfref_market_dfa_export.argtypes = [_P, _P, _P, _P, u32, u32, _P, _P]
        r.mfref_market_language.restype = _I
        r.mfref_market_language.argtypes = [_P, _P, u32, u32, _P, _P]
        _ref = r
    return _ref


def _ptr(a: Optional[np.ndarray]):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle inputs must be C-contiguous"
    return a.ctypes.data


def _c(a, dtype) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=dtype)


# ---------------------------------------------------------------- scalars --

def half_to_float(bits: np.ndarray) -> np.ndarray:
    bits = _c(bits, np.uint16)
    out = np.empty(bits.shape, np.float32)
    lib().orc_half_to_float_n(_ptr(bits), _ptr(out), bits.size)
    return out


def float_to_half_bits(values: np.ndarray) -> np.ndarray:
    values = _c(values, np.float32).ravel()
    f = lib().orc_float_to_half
    return np.array([f(float(v)) for v in values], np.uint16)


# --------------------------------------------------------------- operators --

def rms_norm_f32(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x = _c(x, np.float32)
    w = _c(w, np.float32)
    rows, hidden = x.shape
    y = np.empty_like(x)
    lib().orc_rms_norm_f32(_ptr(x), _ptr(w), eps, _ptr(y), rows, hidden)
    return y


def rms_norm_f16(x_bits: np.ndarray, w_bits: np.ndarray, eps: float) -> np.ndarray:
    x = _c(x_bits, np.uint16)
    w = _c(w_bits, np.uint16)
    rows, hidden = x.shape
    y = np.empty_like(x)
    lib().orc_rms_norm_f16(_ptr(x), _ptr(w), eps, _ptr(y), rows, hidden)
    return y


def dot(hidden: np.ndarray, emb_row_bits: np.ndarray, order: int) -> np.float32:
    h = _c(hidden, np.float32)
    e = _c(emb_row_bits, np.uint16)
    fn = lib().orc_dot_mul_add if order == ORDER_MUL_ADD_CHAIN else lib().orc_dot_fma
    return np.float32(fn(_ptr(h), _ptr(e), h.size))


def scores(hidden: np.ndarray, emb_bits: np.ndarray, tokens: np.ndarray,
           order: int) -> np.ndarray:
    h = _c(hidden, np.float32)
    e = _c(emb_bits, np.uint16)
    t = _c(tokens, np.uint32)
    out = np.empty(t.size, np.float32)
    lib().orc_scores(_ptr(h), _ptr(e), e.shape[1], _ptr(t), t.size, order, _ptr(out))
    return out


def greedy_f16(logits_bits: np.ndarray) -> np.ndarray:
    l = _c(logits_bits, np.uint16)
    rows, vocab = l.shape
    out = np.empty(rows, np.uint32)
    lib().orc_greedy_f16(_ptr(l), rows, vocab, _ptr(out))
    return out


def greedy_f32(logits: np.ndarray) -> np.ndarray:
    l = _c(logits, np.float32)
    rows, vocab = l.shape
    out = np.empty(rows, np.uint32)
    lib().orc_greedy_f32(_ptr(l), rows, vocab, _ptr(out))
    return out


def restricted_greedy_f32(logits, allowed, counts, max_allowed) -> np.ndarray:
    l = _c(logits, np.float32)
    a = _c(allowed, np.uint32)
    c = _c(counts, np.uint32)
    rows, vocab = l.shape
    out = np.empty(rows, np.uint32)
    lib().orc_restricted_greedy_f32(_ptr(l), _ptr(a), _ptr(c), rows, vocab,
                                    max_allowed, _ptr(out))
    return out


def restricted_greedy_f16(logits_bits, allowed, counts, max_allowed) -> np.ndarray:
    l = _c(logits_bits, np.uint16)
    a = _c(allowed, np.uint32)
    c = _c(counts, np.uint32)
    rows, vocab = l.shape
    out = np.empty(rows, np.uint32)
    lib().orc_restricted_greedy_f16(_ptr(l), _ptr(a), _ptr(c), rows, vocab,
                                    max_allowed, _ptr(out))
    return out


def restricted_output_head_f16(hidden_bits, emb_bits, allowed, counts,
                               max_allowed):
    h = _c(hidden_bits, np.uint16)
    e = _c(emb_bits, np.uint16)
    a = _c(allowed, np.uint32)
    c = _c(counts, np.uint32)
    rows, hidden = h.shape
    vocab = e.shape[0]
    tok = np.empty(rows, np.uint32)
    sc = np.empty(rows, np.float32)
    lib().orc_restricted_output_head_f16(_ptr(h), _ptr(e), _ptr(a), _ptr(c), rows,
                                         hidden, vocab, max_allowed, _ptr(tok),
                                         _ptr(sc))
    return tok, sc


def linear_f16(input_bits, weight_bits):
    x = _c(input_bits, np.uint16)
    w = _c(weight_bits, np.uint16)
    rows, inf = x.shape
    outf = w.shape[0]
    out = np.empty((rows, outf), np.uint16)
    out32 = np.empty((rows, outf), np.float32)
    lib().orc_linear_f16(_ptr(x), _ptr(w), rows, inf, outf, _ptr(out), _ptr(out32))
    return out, out32


def decode_tail(x, norm_weight, eps, emb_bits, row_state, state_offsets,
                state_tokens, state_next=None, next_table=None,
                order=ORDER_FMA_CHAIN, threads=1):
    """RMSNorm -> restricted scores -> selection -> DFA advance, per row.

    ``emb_bits`` is a uint16 FP16 table or a float32 table (cfg1).
    ``norm_weight=None`` skips the norm (x is already normalized)."""
    x = _c(x, np.float32)
    nw = None if norm_weight is None else _c(norm_weight, np.float32)
    emb = np.asarray(emb_bits)
    e16 = _c(emb, np.uint16) if emb.dtype != np.float32 else None
    e32 = _c(emb, np.float32) if emb.dtype == np.float32 else None
    rs = _c(row_state, np.uint32)
    so = _c(state_offsets, np.uint32)
    st = _c(state_tokens, np.uint32)
    sn = None if state_next is None else _c(state_next, np.uint32)
    nt = None if next_table is None else _c(next_table, np.int32)
    rows, hidden = x.shape
    vocab = emb.shape[0]
    states = so.size - 1
    tok = np.empty(rows, np.uint32)
    sc = np.empty(rows, np.float32)
    nx = np.empty(rows, np.uint32)
    lib().orc_decode_tail(_ptr(x), _ptr(nw), eps, _ptr(e16), _ptr(e32), vocab,
                          hidden, _ptr(rs),
                          rows, _ptr(so), _ptr(st), states, _ptr(sn), _ptr(nt),
                          order, _ptr(tok), _ptr(sc), _ptr(nx), threads)
    return tok, sc, nx


def decode_tail_sequences(x, norm_weight, eps, emb_bits, table, row_sequence,
                          state_offsets, state_tokens, state_next=None, next_table=None,
                          order=ORDER_FMA_CHAIN, hold=False, threads=1):
    """The decode tail over a per-sequence state table, with the device
    library's conventions for it (the "Sequence table" and
    MF_TAIL_HOLD_FINISHED of include/marketforge_hip.h), restated around
    ``decode_tail``:

    * row r uses the state table[row_sequence[r]] (``row_sequence=None``: row
      r uses table[r]); an index outside the table makes the row invalid and
      writes nothing back;
    * the next states are written back to the same indices of a copy of the
      table, which is returned;
    * ``hold``: a row whose state has an empty list keeps that state.

    Returns (tokens, scores, updated table)."""
    table = np.array(table, dtype=np.uint32)
    rows = np.asarray(x).shape[0]
    seq = np.arange(rows, dtype=np.uint64) if row_sequence is None else \
        np.asarray(row_sequence, dtype=np.uint64)
    inside = seq < table.size
    states = np.full(rows, 0xFFFFFFFF, np.uint32)
    states[inside] = table[seq[inside]]
    tok, sc, nx = decode_tail(x, norm_weight, eps, emb_bits, states, state_offsets,
                              state_tokens, state_next=state_next, next_table=next_table,
                              order=order, threads=threads)
    if hold:
        so = np.asarray(state_offsets, dtype=np.uint32)
        known = states < so.size - 1
        empty = np.zeros(rows, bool)
        empty[known] = so[states[known] + 1] == so[states[known]]
        nx = np.where(empty, states, nx)
    table[seq[inside]] = nx[inside]
    return tok, sc, table
