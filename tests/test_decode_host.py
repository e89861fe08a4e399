"""Host-side ordering of the decode loops' workspace (no GPU needed).

The workspace of a pack must be allocated and zero-filled on the loop's own
stream: a fill on the caller's stream would be unordered with the tail's
kernels on the loop's stream and could overwrite the records of a pack in
flight.  torch and the C ABI are replaced by recorders here, so the test
checks the calls and the stream each one runs under.
"""
import contextlib
import types

import pytest

from market_sim_amd import decode, ops


class FakeTensor:
    def __init__(self, n, log):
        self.n = n
        self.log = log
        self.recorded = []

    def data_ptr(self):
        return 0x10000 + 0x40   # not 256-aligned: the buffer is offset

    def record_stream(self, s):
        self.recorded.append(s)
        self.log.append(("record_stream", s.name))


class FakeStream:
    def __init__(self, name):
        self.name = name
        self.cuda_stream = hash(name) & 0xFFFF


@pytest.fixture
def recorder(monkeypatch):
    import torch
    log = []
    current = {"stream": "caller"}

    @contextlib.contextmanager
    def stream_ctx(s):
        prev = current["stream"]
        current["stream"] = s.name
        try:
            yield
        finally:
            current["stream"] = prev

    def empty(n, dtype=None, device=None):
        log.append(("alloc", current["stream"], n))
        return FakeTensor(n, log)

    def zeros(*a, **k):
        log.append(("zeros", current["stream"]))
        return FakeTensor(0, log)

    monkeypatch.setattr(torch.cuda, "stream", stream_ctx)
    monkeypatch.setattr(torch, "empty", empty)
    monkeypatch.setattr(torch, "zeros", zeros)
    monkeypatch.setattr(ops, "workspace_init",
                        lambda ws, h: log.append(("init", current["stream"], ws.address, h)) or
                        types.SimpleNamespace(code=0, detail=0))
    return log


def test_stream_workspace_allocates_and_fills_on_the_loop_stream(recorder):
    s = FakeStream("loop")
    t, ws = decode.stream_workspace(4096, s, "cuda")
    assert [e[:2] for e in recorder] == [("alloc", "loop"), ("init", "loop")]
    assert ws.address % 256 == 0 and ws.size_bytes == 4096
    assert recorder[1][3] == s.cuda_stream
    assert not any(e[0] == "zeros" for e in recorder)


def test_packer_grows_its_workspace_on_its_stream(recorder, monkeypatch):
    p = object.__new__(decode.SequencePacker)
    p.stream = FakeStream("pack")
    p.device = "cuda"
    p._ws_t = None
    p._ws_bytes = 0
    need = {"n": 1000}
    monkeypatch.setattr(ops, "decode_tail_workspace_bytes", lambda a: need["n"])
    p._workspace(None)
    first = p._ws_t
    need["n"] = 5000
    p._workspace(None)
    # the old tensor is tied to the stream before it is dropped, and both
    # allocations and fills ran under the packer's stream
    assert first.recorded and first.recorded[0].name == "pack"
    kinds = [e for e in recorder if e[0] in ("alloc", "init", "zeros")]
    assert [e[:2] for e in kinds] == [("alloc", "pack"), ("init", "pack"),
                                      ("alloc", "pack"), ("init", "pack")]
    # a smaller pack reuses the workspace
    need["n"] = 100
    p._workspace(None)
    assert len([e for e in recorder if e[0] == "alloc"]) == 2


def test_run_record_of_a_decode_result_passes_the_contract():
    """run_record builds the run contract from a decode result: one request
    per row, tokens up to the row's end, "stop" for rows that reached a
    terminal state, the table named by content."""
    import hashlib
    import os

    import numpy as np

    from market_sim_amd import abi, schema
    from market_sim_amd.dfa import NO_CHOICE
    if not os.path.exists(abi.LIB_PATH):
        pytest.skip("library not built")
    inv = abi.INVALID_TOKEN
    tokens = np.array([[5, 7, 9], [6, 8, inv], [inv, inv, inv]], np.uint32)
    res = decode.DecodeResult(tokens=tokens, scores=np.zeros((3, 3), np.float32),
                              states=np.array([4, 2, 3], np.uint32),
                              choice=np.array([NO_CHOICE, 11, 12], np.uint32))
    table = np.arange(40, dtype=np.uint16).reshape(10, 4)
    rec = decode.run_record(res, [[1], [2, 3], [4]], table, seed=3, inference_seconds=0.25,
                            model_load_seconds=0.5, peak_gpu_memory_bytes=1 << 20,
                            device_name="AMD Instinct MI355X", runtime_version="7.0")
    doc = schema.load_run(rec.to_json())
    assert [r["generated_token_ids"] for r in doc["requests"]] == [[5, 6], [7, 8], [9]]
    assert [r["finish_reason"] for r in doc["requests"]] == ["length", "stop", "stop"]
    assert doc["model"]["checkpoint_sha256"] == hashlib.sha256(table.tobytes()).hexdigest()
    assert doc["metrics"]["output_tokens"] == 5 and doc["metrics"]["input_tokens"] == 4
    assert doc["generation"]["max_output_tokens"] == 3
    with pytest.raises(ValueError):
        decode.run_record(res, [[1]], table, seed=3, inference_seconds=0.25,
                          model_load_seconds=0.5, peak_gpu_memory_bytes=1,
                          device_name="x", runtime_version="7.0")
