"""Device-resident decode tail: uploads a workload once, then runs steps.

Torch CUDA tensors hold the device memory (plumbing only); every computation
goes through the C ABI (``ops.decode_tail_f16`` / ``ops.decode_tail_full_f16``).
"""
from __future__ import annotations

from typing import Optional

import numpy as np

from . import abi, ops, workloads
from .workloads import STATE_UNRESTRICTED, Workload


def _dev(a: np.ndarray, device: str):
    import torch
    a = np.ascontiguousarray(a)
    view = {1: np.int8, 2: np.int16, 4: np.int32}[a.dtype.itemsize] \
        if a.dtype.kind in "ui" else a.dtype
    return torch.from_numpy(a.view(view)).to(device)


class DeviceTail:
    """One workload's tables and buffers on the GPU.

    ``copies`` > 1 keeps that many copies of the embedding table, so timed
    loops can rotate through them and never find the table in the 256 MiB
    Infinity Cache (MALL) from the previous launch."""

    def __init__(self, w: Workload, device: str = "cuda", order: int = abi.ORDER_FMA_CHAIN,
                 copies: int = 1, full: bool = False, advance: Optional[str] = None,
                 unrestricted: Optional[np.ndarray] = None,
                 sorted_lists: Optional[bool] = None, table_pass: bool = False,
                 fused: bool = True, dense: bool = True):
        import torch
        self.w = w
        # MF_TAIL_SORTED_LISTS (the one-pass table kernel where it pays):
        # declared when the lists are strictly ascending (None: checked
        # here) or by the caller; table_pass asks for that kernel even
        # without unrestricted rows.  fused=False keeps packs of short lists
        # off the one-kernel tail (MF_TAIL_NO_FUSED); dense=False keeps long
        # ascending lists on the gather (MF_TAIL_NO_DENSE).
        if sorted_lists is None:
            sorted_lists = workloads.lists_ascending(w.state_offsets, w.state_tokens)
        self.flags = (abi.TAIL_SORTED_LISTS if sorted_lists else 0) | \
            (abi.TAIL_TABLE_PASS if table_pass else 0) | \
            (0 if fused else abi.TAIL_NO_FUSED) | \
            (0 if dense else abi.TAIL_NO_DENSE)
        # the rows handed to the MFMA head (default: the rows whose state is
        # MF_STATE_UNRESTRICTED)
        self._unrestricted = unrestricted
        self.device = device
        self.order = order
        self.stream = torch.cuda.Stream(device=device)
        torch.cuda.synchronize(device)
        with torch.cuda.stream(self.stream):
            self._upload(w, device, copies, full, advance)
        self.stream.synchronize()

    def _upload(self, w: Workload, device: str, copies: int, full: bool,
                advance: Optional[str]) -> None:
        import torch
        self.tables = [_dev(w.embedding, device)]
        for _ in range(copies - 1):
            self.tables.append(self.tables[0].clone())
        self.x = _dev(w.x, device)
        # no weight: x is already normalized (the norm is skipped)
        self.norm_weight = None if w.norm_weight is None else _dev(w.norm_weight, device)
        self.row_state = _dev(w.row_state, device)
        self.offsets = _dev(w.state_offsets, device)
        tokens = w.state_tokens if w.state_tokens.size else np.zeros(1, np.uint32)
        self.tokens = _dev(tokens, device)
        self.state_next = None
        self.next_table = None
        if advance is None:
            advance = "arcs" if w.state_next is not None else (
                "dense" if w.next_table is not None else None)
        if advance == "arcs" and w.state_next is not None:
            self.state_next = _dev(w.state_next, device)
        elif advance == "dense" and w.next_table is not None:
            self.next_table = _dev(w.next_table, device)
        unr = w.unrestricted_rows if self._unrestricted is None else \
            np.asarray(self._unrestricted, dtype=np.uint32)
        self.unrestricted = _dev(unr, device) if unr.size else None
        self.n_unrestricted = int(unr.size)
        B = w.rows
        self.out_token = torch.empty(B, dtype=torch.int32, device=device)
        self.out_score = torch.empty(B, dtype=torch.float32, device=device)
        self.out_next = torch.empty(B, dtype=torch.int32, device=device)
        self.full = full
        args = self.args(0)
        nbytes = ops.decode_tail_workspace_bytes(args, full=full)
        self.workspace = torch.zeros(nbytes // 4 + 64, dtype=torch.int32, device=device)
        # the C ABI wants a 256-byte aligned workspace; torch allocations are
        off = (-self.workspace.data_ptr()) % 256
        self.ws = ops.DeviceBuffer(self.workspace.data_ptr() + off, nbytes)
        abi.check("workspace_init", ops.workspace_init(self.ws, self.stream.cuda_stream))
        self.stream.synchronize()

    def buffers(self, table: int = 0) -> ops.DecodeTailBuffers:
        D = ops.DeviceBuffer.of
        return ops.DecodeTailBuffers(
            x=D(self.x), embedding=D(self.tables[table]), row_state=D(self.row_state),
            state_offsets=D(self.offsets),
            state_tokens=D(self.tokens) if self.w.state_tokens.size else ops.DeviceBuffer(),
            out_token=D(self.out_token), norm_weight=D(self.norm_weight),
            state_next=D(self.state_next), next_table=D(self.next_table),
            unrestricted_rows=D(self.unrestricted), out_score=D(self.out_score),
            out_next_state=D(self.out_next),
            workspace=getattr(self, "ws", ops.DeviceBuffer()))

    def args(self, table: int = 0) -> abi.DecodeTailArgs:
        w = self.w
        return ops.decode_tail_args(
            self.buffers(table), rows=w.rows, hidden=w.hidden, vocab=w.vocab,
            states=w.states, nnz=int(w.state_tokens.size), max_count=w.max_count,
            unrestricted_count=self.n_unrestricted, epsilon=w.epsilon, order=self.order,
            flags=self.flags)

    @property
    def table_pass(self) -> bool:
        """The library runs the one-pass table kernel for this tail."""
        return not self.full and ops.decode_tail_path(self.args(0)) == abi.TAIL_PATH_TABLE_PASS

    @property
    def fused(self) -> bool:
        """The library runs the one-kernel tail (short lists) for this tail."""
        return not self.full and ops.decode_tail_path(self.args(0)) == abi.TAIL_PATH_FUSED

    @property
    def dense(self) -> bool:
        """The unrestricted stage is the dense head."""
        return not self.full and ops.decode_tail_path(self.args(0)) == abi.TAIL_PATH_DENSE

    def launch(self, table: int = 0, args: Optional[abi.DecodeTailArgs] = None) -> None:
        a = args if args is not None else self.args(table)
        fn = ops.decode_tail_full_f16 if self.full else ops.decode_tail_f16
        abi.check("decode_tail", fn(a, self.stream.cuda_stream))

    def set_hidden(self, x: np.ndarray) -> None:
        import torch
        with torch.cuda.stream(self.stream):
            self.x.copy_(_dev(x, self.device))

    def set_state(self, state) -> None:
        """New row states: a host array, or a device tensor (e.g. out_next of
        the previous step, so the DFA state never leaves the GPU)."""
        import torch
        with torch.cuda.stream(self.stream):
            if isinstance(state, np.ndarray):
                self.row_state.copy_(_dev(state, self.device))
            else:
                self.row_state.copy_(state)

    def results(self):
        self.stream.synchronize()
        tok = self.out_token.cpu().numpy().view(np.uint32).copy()
        sc = self.out_score.cpu().numpy().copy()
        nx = self.out_next.cpu().numpy().view(np.uint32).copy()
        return tok, sc, nx

    def run(self, table: int = 0):
        self.launch(table)
        return self.results()
