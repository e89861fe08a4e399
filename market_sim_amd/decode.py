"""Decode loops over the restricted tail, with DFA state resident on the GPU.

The reference generates one restricted token per host round trip:
``CudaSmolLm2::decode_restricted`` (src/cuda/smollm2.cu:336-366, :368-507)
copies the allowed list to the device, runs the norm and the restricted head,
copies the token back and synchronizes; the caller then advances its DFA on
the host (src/grammar/token_dfa.cpp:111-128) and looks up the next list.

Here the DFA lives on the device (``DeviceDfa``), the tail advances it in
the same call that picks the token, and nothing returns to the host until the
caller asks:

* ``RestrictedDecoder`` runs B sequences in lock step: one
  ``mf_decode_tail_f16`` call per step, states alternating between two device
  buffers, every step's tokens kept on the device, finished sequences held in
  their terminal state (``MF_TAIL_HOLD_FINISHED``).  One copy and one
  synchronization per ``result()``, not per token.
* ``SequencePacker`` serves continuous batching: a device table holds the
  DFA state of every resident sequence, and each batch the scheduler forms
  (``InferenceBatch`` of BatchItem{id, work, context_tokens, slot},
  include/marketforge/serving/sequence_scheduler.hpp:36-49) runs as one pack
  whose row r reads and updates the state of the sequence in slot r, in place
  (the C ABI's sequence table).  Only the B slot indices cross PCIe, and only
  when the batch's membership changes.

Torch tensors hold device memory and streams (plumbing); all computation is
the C ABI.
"""
from __future__ import annotations

import os
import re
from dataclasses import dataclass
from typing import Dict, Iterable, List, Optional, Sequence, Tuple

import numpy as np

from . import abi, ops, schema
from .dfa import NO_CHOICE, DfaTables


def _device_u32(a: np.ndarray, device: str):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint32).view(np.int32)).to(device)


def stream_workspace(nbytes: int, stream, device: str):
    """A decode-tail workspace of ``nbytes`` (256-byte aligned) for work on
    ``stream``: allocated under that stream, so torch's allocator orders it
    with the stream's work, and zero-filled there by mf_workspace_init (no
    fill on another stream can overlap the tail).  Returns (tensor, buffer)."""
    import torch
    with torch.cuda.stream(stream):
        t = torch.empty(nbytes // 4 + 64, dtype=torch.int32, device=device)
        off = (-t.data_ptr()) % 256
        ws = ops.DeviceBuffer(t.data_ptr() + off, nbytes)
        abi.check("workspace_init", ops.workspace_init(ws, stream.cuda_stream))
    return t, ws


def _table_tensor(table, device: str):
    """An FP16 [V, H] table as a device tensor (uint16 bits or float16)."""
    import torch
    if isinstance(table, torch.Tensor):
        return table
    return torch.from_numpy(np.ascontiguousarray(table).view(np.int16)).to(device)


class DeviceDfa:
    """A token DFA's CSR export on the device: offsets, arc tokens and arc
    next states (the decode tail's state_offsets / state_tokens /
    state_next); the terminal choices stay on the host."""

    def __init__(self, tables: DfaTables, device: str = "cuda"):
        self.tables = tables
        self.device = device
        self.offsets = _device_u32(tables.offsets, device)
        # a zero-arc DFA still needs a valid token buffer address
        self.tokens = _device_u32(tables.tokens if tables.arcs else np.zeros(1, np.uint32), device)
        self.next = _device_u32(tables.next if tables.arcs else np.zeros(1, np.uint32), device)

    @property
    def states(self) -> int:
        return self.tables.states

    @property
    def nnz(self) -> int:
        return self.tables.arcs

    @property
    def max_count(self) -> int:
        return self.tables.max_count


@dataclass
class DecodeResult:
    """Outcome of a decode loop.

    tokens  u32 [steps, B]: step k's token per row (MF_INVALID_TOKEN once the
            row has finished, or for an invalid row);
    scores  f32 [steps, B]: the chosen tokens' reference-order scores;
    states  u32 [B]: the final DFA state of each row;
    choice  u32 [B]: the terminal choice of the final state (NO_CHOICE when
            the row has not finished)."""
    tokens: np.ndarray
    scores: np.ndarray
    states: np.ndarray
    choice: np.ndarray

    @property
    def finished(self) -> np.ndarray:
        return self.choice != NO_CHOICE

    def generated(self, row: int) -> List[int]:
        """Row ``row``'s tokens up to its end."""
        col = self.tokens[:, row]
        stop = np.nonzero(col == abi.INVALID_TOKEN)[0]
        return col[: stop[0] if stop.size else col.size].tolist()


class RestrictedDecoder:
    """Greedy restricted decoding of ``rows`` sequences in lock step.

    ``step(hidden)`` takes the model's last hidden rows for this step (FP32
    [rows, H] on the device, pre-norm when ``norm_weight`` is given) and
    enqueues one decode-tail call; it never synchronizes.  ``result()``
    synchronizes once and returns every step's tokens."""

    def __init__(self, embedding, dfa: DeviceDfa, rows: int, max_steps: int,
                 norm_weight: Optional[np.ndarray] = None, epsilon: float = 1e-5,
                 order: int = abi.ORDER_FMA_CHAIN, device: str = "cuda", stream=None,
                 fused: bool = True):
        import torch
        # fused=False: the separate kernels even where the one-kernel tail
        # applies (MF_TAIL_NO_FUSED)
        self.flags = abi.TAIL_HOLD_FINISHED | (0 if fused else abi.TAIL_NO_FUSED)
        self.dfa = dfa
        self.device = device
        self.rows = rows
        self.max_steps = max_steps
        self.epsilon = epsilon
        self.order = order
        self.stream = stream if stream is not None else torch.cuda.Stream(device=device)
        self.table = _table_tensor(embedding, device)
        self.vocab, self.hidden = int(self.table.shape[0]), int(self.table.shape[1])
        self.norm_weight = None if norm_weight is None else torch.from_numpy(
            np.ascontiguousarray(norm_weight, dtype=np.float32)).to(device)
        self.states = torch.zeros((2, rows), dtype=torch.int32, device=device)
        self.tokens = torch.empty((max_steps, rows), dtype=torch.int32, device=device)
        self.scores = torch.empty((max_steps, rows), dtype=torch.float32, device=device)
        self._x = torch.empty((rows, self.hidden), dtype=torch.float32, device=device)
        self._args = [self._make_args(k) for k in range(2)]
        nbytes = ops.decode_tail_workspace_bytes(self._args[0])
        self._ws_t, ws = stream_workspace(nbytes, self.stream, device)
        for a in self._args:
            a.workspace = ws.c()
        self.k = 0

    def _make_args(self, parity: int) -> abi.DecodeTailArgs:
        D = ops.DeviceBuffer.of
        b = ops.DecodeTailBuffers(
            x=D(self._x), embedding=D(self.table), row_state=D(self.states[parity]),
            state_offsets=D(self.dfa.offsets), state_tokens=D(self.dfa.tokens),
            out_token=D(self.tokens[0]), norm_weight=D(self.norm_weight),
            state_next=D(self.dfa.next), out_score=D(self.scores[0]),
            out_next_state=D(self.states[1 - parity]))
        return ops.decode_tail_args(
            b, rows=self.rows, hidden=self.hidden, vocab=self.vocab, states=self.dfa.states,
            nnz=self.dfa.nnz, max_count=self.dfa.max_count, epsilon=self.epsilon,
            order=self.order, flags=self.flags)

    def start(self, states: Optional[Sequence[int]] = None) -> None:
        """Every row at the DFA root, or at the given states (one upload)."""
        import torch
        init = np.zeros(self.rows, np.uint32) if states is None else \
            np.asarray(states, dtype=np.uint32)
        with torch.cuda.stream(self.stream):
            self.states[0].copy_(_device_u32(init, self.device))
        self.k = 0

    def step(self, hidden) -> None:
        """One decode step for every row; ``hidden`` is a device FP32
        [rows, H] tensor, read directly (it must stay alive until the step
        has run on the stream)."""
        if self.k >= self.max_steps:
            raise RuntimeError(f"decoder holds {self.max_steps} steps")
        if tuple(hidden.shape) != (self.rows, self.hidden) or not hidden.is_contiguous():
            raise ValueError(f"hidden must be a contiguous [{self.rows}, {self.hidden}] tensor")
        import torch
        # the step runs after the work that produced ``hidden`` on the
        # caller's stream, and the allocator keeps ``hidden`` for this stream
        self.stream.wait_stream(torch.cuda.current_stream(self.device))
        hidden.record_stream(self.stream)
        a = self._args[self.k % 2]
        a.x = ops.DeviceBuffer.of(hidden).c()
        a.out_token = ops.DeviceBuffer.of(self.tokens[self.k]).c()
        a.out_score = ops.DeviceBuffer.of(self.scores[self.k]).c()
        abi.check("decode_tail", ops.decode_tail_f16(a, self.stream.cuda_stream))
        self.k += 1

    def current_states(self):
        """The device tensor holding the states after the last step."""
        return self.states[self.k % 2]

    def result(self) -> DecodeResult:
        self.stream.synchronize()
        k = self.k
        tok = self.tokens[:k].cpu().numpy().view(np.uint32).copy()
        sc = self.scores[:k].cpu().numpy().copy()
        st = self.current_states().cpu().numpy().view(np.uint32).copy()
        choice = np.full(self.rows, NO_CHOICE, np.uint32)
        known = st < self.dfa.states
        choice[known] = self.dfa.tables.choice[st[known]]
        return DecodeResult(tok, sc, st, choice)


# ---- the run contract of a decode run ---------------------------------------

def source_identity() -> Tuple[str, str]:
    """(commit, bundle_sha256) for the run contract's ``source`` block: the
    git commit of this checkout (or, in a snapshot without git history, the
    SHA-1 of the library's sources, a 40-hex content id of the same form),
    and the SHA-256 of the library file that ran."""
    import hashlib
    import subprocess
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    commit = ""
    try:
        r = subprocess.run(["git", "-C", root, "rev-parse", "HEAD"], capture_output=True,
                           text=True, timeout=10, check=False)
        commit = r.stdout.strip() if r.returncode == 0 else ""
    except (OSError, subprocess.SubprocessError):
        commit = ""
    if not re.fullmatch(r"[0-9a-f]{40}", commit):
        h = hashlib.sha1()
        csrc = os.path.join(root, "market_sim_amd", "csrc")
        for name in sorted(os.listdir(csrc)):
            path = os.path.join(csrc, name)
            if os.path.isfile(path):
                h.update(name.encode())
                with open(path, "rb") as f:
                    h.update(f.read())
        commit = h.hexdigest()
    with open(abi.LIB_PATH, "rb") as f:
        bundle = hashlib.sha256(f.read()).hexdigest()
    return commit, bundle


def run_record(result: "DecodeResult", prompts: Sequence[Sequence[int]], table: np.ndarray, *,
               seed: int, inference_seconds: float, model_load_seconds: float,
               peak_gpu_memory_bytes: int, device_name: str, runtime_version: str,
               backend_mode: str = "eager", graphs: bool = False,
               model_id: str = "synthetic-tied-embedding",
               model_repository: str = "local/synthetic") -> schema.RunRecord:
    """The run contract (tools/inference/contract.py:85-160) of a decode run:
    one request per row, its prompt ``prompts[r]`` and the tokens the device
    generated up to the row's end (``DecodeResult.generated``); the finish
    reason is "stop" when the row reached a terminal DFA state, else
    "length".  The model block names the embedding table by content: its
    SHA-256 as checkpoint digest and its SHA-1 as revision.  Generation is
    greedy FP16-table decoding with structured (DFA-restricted) output;
    MI355X (gfx950) reports compute capability 9.5."""
    import hashlib
    tbl = np.ascontiguousarray(table)
    steps, rows = result.tokens.shape
    if len(prompts) != rows:
        raise ValueError(f"{rows} rows need {rows} prompts")
    reqs = tuple(schema.RequestRecord(
        f"seq-{r}", tuple(int(t) for t in prompts[r]), tuple(result.generated(r)),
        "stop" if bool(result.finished[r]) else "length") for r in range(rows))
    commit, bundle = source_identity()
    return schema.RunRecord(
        commit=commit, bundle_sha256=bundle, backend_name="market_sim_amd",
        backend_version=f"abi-{abi.ABI_VERSION}", backend_mode=backend_mode,
        model_id=model_id, model_repository=model_repository,
        model_revision=hashlib.sha1(tbl.tobytes()).hexdigest(),
        checkpoint_sha256=hashlib.sha256(tbl.tobytes()).hexdigest(),
        vocabulary_size=int(tbl.shape[0]), device_name=device_name,
        compute_capability="9.5", runtime_version=runtime_version, dtype="float16",
        seed=int(seed), max_output_tokens=int(steps), requests=reqs,
        model_load_seconds=float(model_load_seconds),
        inference_seconds=float(inference_seconds),
        peak_gpu_memory_bytes=int(peak_gpu_memory_bytes), graphs=graphs,
        structured_output=True)


# ---- continuous batching ----------------------------------------------------

WORK_PREFILL = 0   # serving::WorkKind (sequence_scheduler.hpp:24-27)
WORK_DECODE = 1


@dataclass(frozen=True)
class BatchItem:
    """serving::BatchItem (sequence_scheduler.hpp:36-43)."""
    id: int
    work: int
    context_tokens: int
    slot: int


@dataclass
class PackStep:
    """What one pack produced, per batch slot."""
    ids: List[int]
    tokens: np.ndarray        # u32 [B]
    scores: np.ndarray        # f32 [B]
    states: np.ndarray        # u32 [B] state after the step
    terminal: np.ndarray      # bool [B]: the sequence reached a terminal state
    choice: np.ndarray        # u32 [B]: its terminal choice (NO_CHOICE otherwise)


class SequencePacker:
    """Runs scheduler batches through the decode tail with every resident
    sequence's DFA state in one device table.

    ``admit(id)`` gives a sequence a table entry (at the DFA root, or a given
    state; restricted or unrestricted); ``run(items, hidden)`` packs one
    InferenceBatch (items in slot order, hidden rows in the same order) and
    updates the states in place; ``release(id)`` frees the entry when the
    scheduler retires the sequence.  ``run`` returns the tokens and, per
    slot, whether the sequence reached a terminal state -- the ``terminal``
    argument of SequenceScheduler::complete (sequence_scheduler.hpp:82-84)."""

    def __init__(self, embedding, dfa: DeviceDfa, capacity: int, max_rows: int,
                 norm_weight: Optional[np.ndarray] = None, epsilon: float = 1e-5,
                 order: int = abi.ORDER_FMA_CHAIN, device: str = "cuda", stream=None):
        import torch
        self.dfa = dfa
        self.device = device
        self.capacity = capacity
        self.max_rows = max_rows
        self.epsilon = epsilon
        self.order = order
        self.stream = stream if stream is not None else torch.cuda.Stream(device=device)
        self.table = _table_tensor(embedding, device)
        self.vocab, self.hidden = int(self.table.shape[0]), int(self.table.shape[1])
        self.norm_weight = None if norm_weight is None else torch.from_numpy(
            np.ascontiguousarray(norm_weight, dtype=np.float32)).to(device)
        self.state = torch.zeros(capacity, dtype=torch.int32, device=device)
        self.row_sequence = torch.zeros(max_rows, dtype=torch.int32, device=device)
        self.unrestricted = torch.zeros(max_rows, dtype=torch.int32, device=device)
        self.out_token = torch.empty(max_rows, dtype=torch.int32, device=device)
        self.out_score = torch.empty(max_rows, dtype=torch.float32, device=device)
        self._entry: Dict[int, int] = {}
        self._free = list(range(capacity - 1, -1, -1))
        self._unrestricted_ids = set()
        self._last_pack: Optional[tuple] = None
        self._ws_t = None
        self._ws_bytes = 0

    # -- residency ------------------------------------------------------------
    def admit(self, seq_id: int, state: int = 0, unrestricted: bool = False) -> int:
        """Gives ``seq_id`` a table entry holding ``state`` (or the
        unrestricted marker); returns the entry."""
        import torch
        if seq_id in self._entry:
            raise ValueError(f"sequence {seq_id} is already resident")
        if not self._free:
            raise RuntimeError("the state table is full")
        e = self._free.pop()
        self._entry[seq_id] = e
        value = abi.STATE_UNRESTRICTED if unrestricted else state
        if unrestricted:
            self._unrestricted_ids.add(seq_id)
        with torch.cuda.stream(self.stream):
            self.state[e].fill_(np.uint32(value).view(np.int32).item())
        return e

    def release(self, seq_id: int) -> None:
        e = self._entry.pop(seq_id)
        self._unrestricted_ids.discard(seq_id)
        self._free.append(e)

    def resident(self) -> int:
        return len(self._entry)

    # -- one pack -------------------------------------------------------------
    def _workspace(self, args: abi.DecodeTailArgs) -> ops.DeviceBuffer:
        """The pack's workspace, grown when a pack needs more.  Called after
        the stream has waited for the caller's stream; the replaced tensor
        is marked as used by the stream, so its memory is not handed out
        again before a pack still in flight (run(sync=False)) is done."""
        need = ops.decode_tail_workspace_bytes(args)
        if need > self._ws_bytes:
            if self._ws_t is not None:
                self._ws_t.record_stream(self.stream)
            self._ws_t, self._ws = stream_workspace(need, self.stream, self.device)
            self._ws_bytes = need
        return self._ws

    def run(self, items: Sequence[BatchItem], hidden, sync: bool = True) -> Optional[PackStep]:
        """One decode-tail call for the batch: row r is the sequence of
        ``items[r]`` (slots 0..B-1 in order) and reads ``hidden[r]``."""
        import torch
        B = len(items)
        if B == 0 or B > self.max_rows:
            raise ValueError(f"a pack holds 1..{self.max_rows} rows")
        if any(it.slot != r for r, it in enumerate(items)):
            raise ValueError("batch items must be in slot order")
        if tuple(hidden.shape) != (B, self.hidden) or not hidden.is_contiguous():
            raise ValueError(f"hidden must be a contiguous [{B}, {self.hidden}] tensor")
        ids = [it.id for it in items]
        entries = [self._entry[i] for i in ids]   # KeyError: not admitted
        if len(set(entries)) != B:
            raise ValueError("a sequence appears twice in the batch")
        unr = [r for r, i in enumerate(ids) if i in self._unrestricted_ids]
        key = (tuple(entries), tuple(unr))
        self.stream.wait_stream(torch.cuda.current_stream(self.device))
        hidden.record_stream(self.stream)
        with torch.cuda.stream(self.stream):
            if key != self._last_pack:
                # the pack's membership changed: B slot indices go up
                self.row_sequence[:B].copy_(_device_u32(np.array(entries), self.device))
                if unr:
                    self.unrestricted[:len(unr)].copy_(_device_u32(np.array(unr), self.device))
                self._last_pack = key
        D = ops.DeviceBuffer.of
        b = ops.DecodeTailBuffers(
            x=D(hidden), embedding=D(self.table), row_state=D(self.state),
            state_offsets=D(self.dfa.offsets), state_tokens=D(self.dfa.tokens),
            out_token=D(self.out_token[:B]), norm_weight=D(self.norm_weight),
            state_next=D(self.dfa.next), out_score=D(self.out_score[:B]),
            out_next_state=D(self.state), row_sequence=D(self.row_sequence[:B]),
            unrestricted_rows=D(self.unrestricted[:len(unr)]) if unr else ops.DeviceBuffer())
        a = ops.decode_tail_args(b, rows=B, hidden=self.hidden, vocab=self.vocab,
                                 states=self.dfa.states, nnz=self.dfa.nnz,
                                 max_count=self.dfa.max_count, unrestricted_count=len(unr),
                                 epsilon=self.epsilon, order=self.order,
                                 flags=abi.TAIL_HOLD_FINISHED)
        a.workspace = self._workspace(a).c()
        abi.check("decode_tail", ops.decode_tail_f16(a, self.stream.cuda_stream))
        if not sync:
            return None
        return self.collect(ids)

    def collect(self, ids: Sequence[int]) -> PackStep:
        """Synchronizes and reads the last pack's outputs."""
        B = len(ids)
        self.stream.synchronize()
        tok = self.out_token[:B].cpu().numpy().view(np.uint32).copy()
        sc = self.out_score[:B].cpu().numpy().copy()
        table = self.state.cpu().numpy().view(np.uint32)
        st = table[[self._entry[i] for i in ids]].copy()
        choice = np.full(B, NO_CHOICE, np.uint32)
        known = st < self.dfa.states
        choice[known] = self.dfa.tables.choice[st[known]]
        return PackStep(list(ids), tok, sc, st, choice != NO_CHOICE, choice)

    def states_of(self, ids: Iterable[int]) -> np.ndarray:
        self.stream.synchronize()
        table = self.state.cpu().numpy().view(np.uint32)
        return table[[self._entry[i] for i in ids]].copy()
