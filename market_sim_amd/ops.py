"""Python mirror of the reference operator API over the C ABI.

Same names, argument meaning and error behaviour as
include/marketforge/cuda/{greedy,rms_norm,linear}.hpp: every op takes
device buffers (``DeviceBuffer``: address + size in bytes, the reference's
DeviceBuffer view), explicit shape arguments and a stream, validates before
launching, and returns a ``Status`` (code + detail) instead of raising.
Device memory is any torch CUDA tensor (``DeviceBuffer.of``) or a raw
allocation from ``DeviceBuffer.allocate``; torch is plumbing only.
"""
from __future__ import annotations

import ctypes
import dataclasses
from typing import Optional

import numpy as np

from . import abi

Status = abi.Status


@dataclasses.dataclass(frozen=True)
class DeviceBuffer:
    """(address, size_bytes): include/marketforge/cuda/device_buffer.hpp:20-56."""
    address: int = 0
    size_bytes: int = 0

    @staticmethod
    def of(tensor) -> "DeviceBuffer":
        if tensor is None:
            return DeviceBuffer()
        return DeviceBuffer(int(tensor.data_ptr()), int(tensor.numel() * tensor.element_size()))

    def c(self) -> abi.Buffer:
        return abi.Buffer(self.address, self.size_bytes)


def allocate(nbytes: int) -> DeviceBuffer:
    """DeviceBuffer::allocate (src/cuda/device_buffer.cu:36-55)."""
    addr = ctypes.c_size_t()
    abi.check("mf_device_alloc", abi.lib().mf_device_alloc(nbytes, ctypes.byref(addr)))
    return DeviceBuffer(addr.value, nbytes)


def free(buffer: DeviceBuffer) -> Status:
    return abi.lib().mf_device_free(buffer.address)


def stream_create() -> int:
    s = ctypes.c_size_t()
    abi.check("mf_stream_create", abi.lib().mf_stream_create(ctypes.byref(s)))
    return s.value


def stream_synchronize(stream: int) -> Status:
    return abi.lib().mf_stream_synchronize(stream)


def stream_destroy(stream: int) -> Status:
    return abi.lib().mf_stream_destroy(stream)


def copy_from_host_async(dst: DeviceBuffer, host: np.ndarray, offset: int,
                         stream: int) -> Status:
    host = np.ascontiguousarray(host)
    return abi.lib().mf_copy_to_device_async(dst.c(), offset, host.ctypes.data,
                                            host.nbytes, stream)


def copy_to_host_async(host: np.ndarray, src: DeviceBuffer, offset: int,
                       stream: int) -> Status:
    assert host.flags["C_CONTIGUOUS"]
    return abi.lib().mf_copy_to_host_async(host.ctypes.data, src.c(), offset,
                                          host.nbytes, stream)


# ------------------------------------------------------ reference operators --

def rms_norm_f32(input: DeviceBuffer, weight: DeviceBuffer, output: DeviceBuffer,
                 rows: int, hidden_size: int, epsilon: float, stream: int) -> Status:
    """include/marketforge/cuda/rms_norm.hpp:18-22."""
    return abi.lib().mf_rms_norm_f32(input.c(), weight.c(), output.c(), rows,
                                    hidden_size, epsilon, stream)


def rms_norm_f16(input: DeviceBuffer, weight: DeviceBuffer, output: DeviceBuffer,
                 rows: int, hidden_size: int, epsilon: float, stream: int) -> Status:
    """include/marketforge/cuda/rms_norm.hpp:24-28."""
    return abi.lib().mf_rms_norm_f16(input.c(), weight.c(), output.c(), rows,
                                    hidden_size, epsilon, stream)


def greedy_select_f16(logits: DeviceBuffer, token_ids: DeviceBuffer, rows: int,
                      vocabulary_size: int, stream: int) -> Status:
    """include/marketforge/cuda/greedy.hpp:17-21."""
    return abi.lib().mf_greedy_select_f16(logits.c(), token_ids.c(), rows,
                                         vocabulary_size, stream)


def greedy_select_f32(logits: DeviceBuffer, token_ids: DeviceBuffer, rows: int,
                      vocabulary_size: int, stream: int) -> Status:
    return abi.lib().mf_greedy_select_f32(logits.c(), token_ids.c(), rows,
                                         vocabulary_size, stream)


def restricted_greedy_select_f16(logits: DeviceBuffer, allowed_token_ids: DeviceBuffer,
                                 allowed_token_counts: DeviceBuffer,
                                 token_ids: DeviceBuffer, rows: int,
                                 vocabulary_size: int, maximum_allowed_tokens: int,
                                 stream: int) -> Status:
    """include/marketforge/cuda/greedy.hpp:29-33."""
    return abi.lib().mf_restricted_greedy_select_f16(
        logits.c(), allowed_token_ids.c(), allowed_token_counts.c(), token_ids.c(),
        rows, vocabulary_size, maximum_allowed_tokens, stream)


def restricted_greedy_select_f32(logits, allowed_token_ids, allowed_token_counts,
                                 token_ids, rows, vocabulary_size,
                                 maximum_allowed_tokens, stream) -> Status:
    return abi.lib().mf_restricted_greedy_select_f32(
        logits.c(), allowed_token_ids.c(), allowed_token_counts.c(), token_ids.c(),
        rows, vocabulary_size, maximum_allowed_tokens, stream)


def restricted_output_head_f16(hidden: DeviceBuffer, embedding: DeviceBuffer,
                               allowed_token_ids: DeviceBuffer,
                               allowed_token_counts: DeviceBuffer,
                               token_ids: DeviceBuffer, rows: int, hidden_size: int,
                               vocabulary_size: int, maximum_allowed_tokens: int,
                               stream: int) -> Status:
    """include/marketforge/cuda/greedy.hpp:43-49."""
    return abi.lib().mf_restricted_output_head_f16(
        hidden.c(), embedding.c(), allowed_token_ids.c(), allowed_token_counts.c(),
        token_ids.c(), rows, hidden_size, vocabulary_size, maximum_allowed_tokens,
        stream)


def linear_f16(input: DeviceBuffer, weight: DeviceBuffer, output: DeviceBuffer,
               rows: int, input_features: int, output_features: int,
               stream: int) -> Status:
    """include/marketforge/cuda/linear.hpp:18-22 (no BLAS handle)."""
    return abi.lib().mf_linear_f16(input.c(), weight.c(), output.c(), rows,
                                  input_features, output_features, stream)


# ------------------------------------------------------------- decode tail --

@dataclasses.dataclass
class DecodeTailBuffers:
    """Device buffers of one decode-tail call (see mf_decode_tail_args)."""
    x: DeviceBuffer
    embedding: DeviceBuffer
    row_state: DeviceBuffer
    state_offsets: DeviceBuffer
    state_tokens: DeviceBuffer
    out_token: DeviceBuffer
    norm_weight: DeviceBuffer = DeviceBuffer()
    state_next: DeviceBuffer = DeviceBuffer()
    next_table: DeviceBuffer = DeviceBuffer()
    unrestricted_rows: DeviceBuffer = DeviceBuffer()
    out_score: DeviceBuffer = DeviceBuffer()
    out_next_state: DeviceBuffer = DeviceBuffer()
    workspace: DeviceBuffer = DeviceBuffer()
    row_sequence: DeviceBuffer = DeviceBuffer()


def decode_tail_args(b: DecodeTailBuffers, *, rows: int, hidden: int, vocab: int,
                     states: int, nnz: int, max_count: int,
                     unrestricted_count: int = 0, epsilon: float = 1e-5,
                     order: int = abi.ORDER_FMA_CHAIN, flags: int = 0) -> abi.DecodeTailArgs:
    a = abi.DecodeTailArgs()
    a.x = b.x.c()
    a.norm_weight = b.norm_weight.c()
    a.epsilon = epsilon
    a.order = order
    a.embedding = b.embedding.c()
    a.row_state = b.row_state.c()
    a.state_offsets = b.state_offsets.c()
    a.state_tokens = b.state_tokens.c()
    a.state_next = b.state_next.c()
    a.next_table = b.next_table.c()
    a.unrestricted_rows = b.unrestricted_rows.c()
    a.out_token = b.out_token.c()
    a.out_score = b.out_score.c()
    a.out_next_state = b.out_next_state.c()
    a.workspace = b.workspace.c()
    a.rows, a.hidden, a.vocab, a.states = rows, hidden, vocab, states
    a.nnz, a.max_count, a.unrestricted_count = nnz, max_count, unrestricted_count
    a.row_sequence = b.row_sequence.c()
    a.flags = flags
    return a


def decode_tail_workspace_bytes(args: abi.DecodeTailArgs, full: bool = False) -> int:
    n = ctypes.c_uint64()
    fn = (abi.lib().mf_decode_tail_full_workspace_bytes if full
          else abi.lib().mf_decode_tail_workspace_bytes)
    abi.check("workspace_bytes", fn(ctypes.byref(args), ctypes.byref(n)))
    return n.value


def decode_tail_path(args: abi.DecodeTailArgs) -> int:
    """abi.TAIL_PATH_GATHER, abi.TAIL_PATH_TABLE_PASS, abi.TAIL_PATH_FUSED or
    abi.TAIL_PATH_DENSE: the kernels mf_decode_tail_f16 runs for these arguments."""
    n = ctypes.c_uint32()
    abi.check("decode_tail_path", abi.lib().mf_decode_tail_path(ctypes.byref(args), ctypes.byref(n)))
    return n.value


def workspace_init(workspace: DeviceBuffer, stream: int) -> Status:
    return abi.lib().mf_workspace_init(workspace.c(), stream)


def read_floor(data: DeviceBuffer, sink: DeviceBuffer, stream: int) -> Status:
    return abi.lib().mf_read_floor(data.c(), sink.c(), stream)


def decode_tail_f16(args: abi.DecodeTailArgs, stream: int) -> Status:
    return abi.lib().mf_decode_tail_f16(ctypes.byref(args), stream)


def decode_tail_f16_noalloc(args: abi.DecodeTailArgs, stream: int) -> Status:
    """mf_decode_tail_f16 on the library's own per-GPU workspace (no
    allocation; args.workspace is not used)."""
    return abi.lib().mf_decode_tail_f16_noalloc(ctypes.byref(args), stream)


def decode_tail_noalloc_max_bytes() -> int:
    return int(abi.lib().mf_decode_tail_noalloc_max_bytes())


def decode_tail_prepare(args: abi.DecodeTailArgs, stream: int) -> Status:
    return abi.lib().mf_decode_tail_prepare(ctypes.byref(args), stream)


def decode_tail_restricted(args: abi.DecodeTailArgs, stream: int) -> Status:
    return abi.lib().mf_decode_tail_restricted(ctypes.byref(args), stream)


def decode_tail_unrestricted(args: abi.DecodeTailArgs, stream: int) -> Status:
    return abi.lib().mf_decode_tail_unrestricted(ctypes.byref(args), stream)


def decode_tail_finalize(args: abi.DecodeTailArgs, stream: int) -> Status:
    return abi.lib().mf_decode_tail_finalize(ctypes.byref(args), stream)


def decode_tail_full_f16(args: abi.DecodeTailArgs, stream: int) -> Status:
    return abi.lib().mf_decode_tail_full_f16(ctypes.byref(args), stream)
