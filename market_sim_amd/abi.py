"""ctypes binding of the C ABI in include/marketforge_hip.h.

Loads ``market_sim_amd/lib/libmarketforge_hip.so`` (built in-tree by
``market_sim_amd/build.py``).  There is no CPU fallback: if the library is
missing, ``lib()`` raises.  Device memory and streams are plain integers
(addresses / handles), exactly as the C ABI takes them.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libmarketforge_hip.so")

MF_OK = 0
MF_INVALID_ARGUMENT = 1
MF_UNSUPPORTED_DTYPE = 2
MF_INVALID_SHAPE = 3
MF_ARITHMETIC_OVERFLOW = 5
MF_ALLOCATION_FAILED = 7
MF_RESOURCE_LIMIT = 15
MF_DEVICE_BACKEND_FAILURE = 21
MF_DEVICE_RUNTIME_FAILURE = 22

INVALID_TOKEN = 0xFFFFFFFF
STATE_UNRESTRICTED = 0xFFFFFFFE
STATE_INVALID = 0xFFFFFFFF
ORDER_FMA_CHAIN = 0
ORDER_MUL_ADD_CHAIN = 1
TAIL_HOLD_FINISHED = 1
TAIL_SORTED_LISTS = 2
TAIL_TABLE_PASS = 4
TAIL_NO_FUSED = 8
TAIL_NO_DENSE = 16
TAIL_PATH_GATHER = 0
TAIL_PATH_TABLE_PASS = 1
TAIL_PATH_FUSED = 2
TAIL_PATH_DENSE = 3
ABI_VERSION = 6

_U64 = ctypes.c_uint64
_UP = ctypes.c_size_t  # uintptr_t


class Status(ctypes.Structure):
    _fields_ = [("code", ctypes.c_int32), ("detail", ctypes.c_uint32)]

    def __repr__(self) -> str:
        return f"Status(code={self.code}, detail={self.detail})"


class Buffer(ctypes.Structure):
    """mf_buffer: a device address and its allocation size in bytes."""
    _fields_ = [("address", _UP), ("bytes", _U64)]


class DecodeTailArgs(ctypes.Structure):
    _fields_ = [
        ("x", Buffer), ("norm_weight", Buffer), ("epsilon", ctypes.c_float),
        ("order", ctypes.c_int32), ("embedding", Buffer), ("row_state", Buffer),
        ("state_offsets", Buffer), ("state_tokens", Buffer), ("state_next", Buffer),
        ("next_table", Buffer), ("unrestricted_rows", Buffer), ("out_token", Buffer),
        ("out_score", Buffer), ("out_next_state", Buffer), ("workspace", Buffer),
        ("rows", _U64), ("hidden", _U64), ("vocab", _U64), ("states", _U64),
        ("nnz", _U64), ("max_count", _U64), ("unrestricted_count", _U64),
        ("row_sequence", Buffer), ("flags", _U64),
    ]


# Every exported entry point and its signature (used by the binding and by
# the CPU test that checks the library exports what the header declares).
SIGNATURES = {
    "mf_abi_version": (ctypes.c_uint32, []),
    "mf_device_count": (Status, [ctypes.POINTER(ctypes.c_int32)]),
    "mf_device_alloc": (Status, [_U64, ctypes.POINTER(_UP)]),
    "mf_device_free": (Status, [_UP]),
    "mf_copy_to_device_async": (Status, [Buffer, _U64, ctypes.c_void_p, _U64, _UP]),
    "mf_copy_to_host_async": (Status, [ctypes.c_void_p, Buffer, _U64, _U64, _UP]),
    "mf_stream_create": (Status, [ctypes.POINTER(_UP)]),
    "mf_stream_destroy": (Status, [_UP]),
    "mf_stream_synchronize": (Status, [_UP]),
    "mf_rms_norm_f32": (Status, [Buffer, Buffer, Buffer, _U64, _U64, ctypes.c_float, _UP]),
    "mf_rms_norm_f16": (Status, [Buffer, Buffer, Buffer, _U64, _U64, ctypes.c_float, _UP]),
    "mf_greedy_select_f16": (Status, [Buffer, Buffer, _U64, _U64, _UP]),
    "mf_greedy_select_f32": (Status, [Buffer, Buffer, _U64, _U64, _UP]),
    "mf_restricted_greedy_select_f16": (
        Status, [Buffer, Buffer, Buffer, Buffer, _U64, _U64, _U64, _UP]),
    "mf_restricted_greedy_select_f32": (
        Status, [Buffer, Buffer, Buffer, Buffer, _U64, _U64, _U64, _UP]),
    "mf_restricted_output_head_f16": (
        Status, [Buffer, Buffer, Buffer, Buffer, Buffer, _U64, _U64, _U64, _U64, _UP]),
    "mf_linear_f16": (Status, [Buffer, Buffer, Buffer, _U64, _U64, _U64, _UP]),
    "mf_decode_tail_workspace_bytes": (
        Status, [ctypes.POINTER(DecodeTailArgs), ctypes.POINTER(_U64)]),
    "mf_decode_tail_path": (
        Status, [ctypes.POINTER(DecodeTailArgs), ctypes.POINTER(ctypes.c_uint32)]),
    "mf_workspace_init": (Status, [Buffer, _UP]),
    "mf_read_floor": (Status, [Buffer, Buffer, _UP]),
    "mf_decode_tail_f16": (Status, [ctypes.POINTER(DecodeTailArgs), _UP]),
    "mf_decode_tail_noalloc_max_bytes": (_U64, []),
    "mf_decode_tail_f16_noalloc": (Status, [ctypes.POINTER(DecodeTailArgs), _UP]),
    "mf_decode_tail_prepare": (Status, [ctypes.POINTER(DecodeTailArgs), _UP]),
    "mf_decode_tail_restricted": (Status, [ctypes.POINTER(DecodeTailArgs), _UP]),
    "mf_decode_tail_unrestricted": (Status, [ctypes.POINTER(DecodeTailArgs), _UP]),
    "mf_decode_tail_finalize": (Status, [ctypes.POINTER(DecodeTailArgs), _UP]),
    "mf_decode_tail_full_workspace_bytes": (
        Status, [ctypes.POINTER(DecodeTailArgs), ctypes.POINTER(_U64)]),
    "mf_decode_tail_full_f16": (Status, [ctypes.POINTER(DecodeTailArgs), _UP]),
}

_lib: Optional[ctypes.CDLL] = None


class MarketForgeError(RuntimeError):
    """A non-OK mf_status (the reference's Status{code, detail})."""

    def __init__(self, where: str, status: Status):
        super().__init__(f"{where}: code={status.code} detail={status.detail}")
        self.code = status.code
        self.detail = status.detail


def lib() -> ctypes.CDLL:
    """The HIP library; raises if it has not been built (no fallback)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m market_sim_amd.build`")
        l = ctypes.CDLL(LIB_PATH)
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(l, name)
            fn.restype = restype
            fn.argtypes = argtypes
        if l.mf_abi_version() != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH} has ABI version {l.mf_abi_version()}, this binding "
                               f"expects {ABI_VERSION}: rebuild it")
        _lib = l
    return _lib


def check(where: str, status: Status) -> None:
    if status.code != MF_OK:
        raise MarketForgeError(where, status)


def buf(address: int, nbytes: int) -> Buffer:
    return Buffer(address, nbytes)
