"""Result schemas of the reference, emitted and checked for MI355X runs.

Two documents keep the reference's field sets exactly, so that its tooling
reads ours unchanged:

* the restricted output-head benchmark line written by
  src/tools/cuda_restricted_output_head_bench.cu:300-330 and checked by
  tools/modal/vllm_modal_app.py:459-516 (here: ``check_output_head_benchmark``);
* the inference run contract of tools/inference/contract.py:11-428
  (here: ``RunRecord`` and ``check_run``), the document a decode loop
  reports.

The reference pins its GPU identity (an L4, compute capability "8.9"); the
checks here take the expected identity as arguments instead.  MI355X is
gfx950, which HIP reports as compute capability "9.5" and which the contract's
``cpu|N.N`` pattern (contract.py:15) accepts.
"""
from __future__ import annotations

import json
import math
import re
from dataclasses import dataclass
from typing import Dict, List, Optional, Sequence, Tuple

SCHEMA_VERSION = 1


class SchemaError(ValueError):
    """A document does not match the reference schema (contract.py:21-22)."""


# ---- field checks -----------------------------------------------------------

def _object(value, keys, where: str) -> dict:
    if type(value) is not dict:
        raise SchemaError(f"{where}: expected an object")
    if set(value) != set(keys):
        missing = sorted(set(keys) - set(value))
        extra = sorted(set(value) - set(keys))
        raise SchemaError(f"{where}: fields differ (missing {missing}, unexpected {extra})")
    return value


def _int(value, where: str, lo: int = 0) -> int:
    if type(value) is not int or value < lo:
        raise SchemaError(f"{where}: expected an integer >= {lo}")
    return value


def _float(value, where: str, positive: bool = False) -> float:
    if type(value) is not float or not math.isfinite(value):
        raise SchemaError(f"{where}: expected a finite float")
    if value < 0.0 or (positive and value == 0.0):
        raise SchemaError(f"{where}: expected a {'positive' if positive else 'non-negative'} value")
    return value


def _text(value, where: str) -> str:
    if type(value) is not str or value == "":
        raise SchemaError(f"{where}: expected a non-empty string")
    return value


def _flag(value, where: str) -> bool:
    if type(value) is not bool:
        raise SchemaError(f"{where}: expected a boolean")
    return value


# ---- restricted output-head benchmark --------------------------------------

# The benchmark's fixed shape and case grid
# (src/tools/cuda_restricted_output_head_bench.cu:25-26, :278-291).
HEAD_BENCH_HIDDEN = 576
HEAD_BENCH_VOCAB = 49_152
HEAD_BENCH_ROWS = (1, 16, 256)
HEAD_BENCH_ALLOWED = (2, 8, 32, 128)
_HEAD_BENCH_KEYS = ("schema_version", "result", "operator", "model_shape", "hidden_size",
                    "vocabulary_size", "gpu", "measurements")
_HEAD_CELL_KEYS = ("rows", "allowed_tokens_per_row", "iterations", "full_average_microseconds",
                   "restricted_average_microseconds", "speedup", "full_scores",
                   "restricted_scores", "materialized_logit_bytes_avoided",
                   "exact_token_parity")

# The reference's published NVIDIA L4 cells, (rows, allowed) -> (full us,
# restricted us) (BENCHMARKS.md:33-44).
L4_OUTPUT_HEAD_US: Dict[Tuple[int, int], Tuple[float, float]] = {
    (1, 2): (238.672, 12.872), (1, 8): (238.643, 14.864),
    (1, 32): (238.533, 26.196), (1, 128): (238.635, 44.702),
    (16, 2): (249.651, 13.155), (16, 8): (249.631, 15.012),
    (16, 32): (249.334, 26.423), (16, 128): (248.832, 45.609),
    (256, 2): (365.312, 17.633), (256, 8): (370.473, 28.938),
    (256, 32): (375.009, 91.177), (256, 128): (374.170, 294.144),
}


def check_output_head_benchmark(doc, gpu_name_contains: str = "",
                                compute_capability: Optional[str] = None) -> None:
    """Raises SchemaError unless ``doc`` is a complete output-head benchmark
    document (vllm_modal_app.py:459-516): the fixed identity, all 12 cells
    once each, exact token parity in every cell, positive finite timings and
    the derived counts rows x V, rows x allowed and rows x V x 2."""
    root = _object(doc, _HEAD_BENCH_KEYS, "benchmark")
    if (root["schema_version"] != SCHEMA_VERSION or root["result"] != "pass"
            or root["operator"] != "restricted_output_head_f16"
            or root["model_shape"] != "SmolLM2-135M"
            or root["hidden_size"] != HEAD_BENCH_HIDDEN
            or root["vocabulary_size"] != HEAD_BENCH_VOCAB):
        raise SchemaError("benchmark: identity fields do not match")
    gpu = _object(root["gpu"], ("name", "compute_capability"), "benchmark.gpu")
    if gpu_name_contains not in _text(gpu["name"], "gpu.name"):
        raise SchemaError(f"gpu.name does not name {gpu_name_contains!r}")
    cc = _text(gpu["compute_capability"], "gpu.compute_capability")
    if compute_capability is not None and cc != compute_capability:
        raise SchemaError(f"gpu.compute_capability {cc!r} != {compute_capability!r}")
    cells = root["measurements"]
    if type(cells) is not list or len(cells) != len(HEAD_BENCH_ROWS) * len(HEAD_BENCH_ALLOWED):
        raise SchemaError("benchmark.measurements: expected 12 cells")
    seen = set()
    for i, raw in enumerate(cells):
        where = f"measurements[{i}]"
        cell = _object(raw, _HEAD_CELL_KEYS, where)
        rows = _int(cell["rows"], where + ".rows", 1)
        allowed = _int(cell["allowed_tokens_per_row"], where + ".allowed_tokens_per_row", 1)
        _int(cell["iterations"], where + ".iterations", 1)
        if rows not in HEAD_BENCH_ROWS or allowed not in HEAD_BENCH_ALLOWED:
            raise SchemaError(f"{where}: cell ({rows}, {allowed}) is not in the grid")
        if (cell["full_scores"] != rows * HEAD_BENCH_VOCAB
                or cell["restricted_scores"] != rows * allowed
                or cell["materialized_logit_bytes_avoided"] != rows * HEAD_BENCH_VOCAB * 2):
            raise SchemaError(f"{where}: derived counts do not match the cell")
        if cell["exact_token_parity"] is not True:
            raise SchemaError(f"{where}: token parity failed")
        for k in ("full_average_microseconds", "restricted_average_microseconds", "speedup"):
            _float(cell[k], f"{where}.{k}", positive=True)
        seen.add((rows, allowed))
    if len(seen) != len(cells):
        raise SchemaError("benchmark.measurements: a cell is repeated")


# ---- restricted-greedy and RMSNorm benchmarks --------------------------------

# The documents of the reference's restricted-greedy benchmark
# (src/tools/cuda_restricted_greedy_bench.cu:262-296, validated by
# tools/modal/vllm_modal_app.py:359-427) and RMSNorm benchmark
# (src/tools/cuda_rmsnorm_bench.cu:155-175, vllm_modal_app.py:283-356):
# exactly these fields, positive counts, positive finite rates.
_GREEDY_BENCH_KEYS = ("schema_version", "result", "operator", "grammar", "vocabulary_size",
                      "grammar_states", "grammar_arcs", "maximum_allowed_tokens", "gpu",
                      "measurements")
_GREEDY_CELL_KEYS = ("rows", "total_allowed_candidates", "iterations", "average_microseconds",
                     "sequences_per_second", "candidate_gib_per_second")
GREEDY_BENCH_ROWS = (1, 16, 256)
_NORM_BENCH_KEYS = ("schema_version", "result", "operator", "model_shape", "gpu", "measurements")
_NORM_CELL_KEYS = ("rows", "hidden_size", "iterations", "average_microseconds",
                   "logical_gib_per_second")
NORM_BENCH_ROWS = (1, 16, 256, 1024)


def check_restricted_greedy_benchmark(doc) -> None:
    """Raises SchemaError unless ``doc`` is a restricted-greedy benchmark
    document with the reference's fields and values (apart from the GPU
    identity, which names the device it ran on)."""
    root = _object(doc, _GREEDY_BENCH_KEYS, "benchmark")
    if (root["schema_version"] != SCHEMA_VERSION or root["result"] != "pass"
            or root["operator"] != "restricted_greedy_f16"
            or root["grammar"] != "smollm2_market_action_v1"
            or root["vocabulary_size"] != HEAD_BENCH_VOCAB):
        raise SchemaError("benchmark: identity fields do not match")
    for k in ("grammar_states", "grammar_arcs", "maximum_allowed_tokens"):
        _int(root[k], f"benchmark.{k}", 1)
    gpu = _object(root["gpu"], ("name", "compute_capability"), "benchmark.gpu")
    _text(gpu["name"], "gpu.name")
    _text(gpu["compute_capability"], "gpu.compute_capability")
    cells = root["measurements"]
    if type(cells) is not list or len(cells) != len(GREEDY_BENCH_ROWS):
        raise SchemaError("benchmark.measurements: expected 3 cases")
    for i, raw in enumerate(cells):
        where = f"measurements[{i}]"
        cell = _object(raw, _GREEDY_CELL_KEYS, where)
        if _int(cell["rows"], where + ".rows", 1) != GREEDY_BENCH_ROWS[i]:
            raise SchemaError(f"{where}: rows {cell['rows']} out of order")
        _int(cell["total_allowed_candidates"], where + ".total_allowed_candidates", 1)
        _int(cell["iterations"], where + ".iterations", 1)
        for k in ("average_microseconds", "sequences_per_second", "candidate_gib_per_second"):
            _float(cell[k], f"{where}.{k}", positive=True)


def check_rmsnorm_benchmark(doc) -> None:
    """Raises SchemaError unless ``doc`` is an RMSNorm benchmark document
    with the reference's fields and values (apart from the GPU identity)."""
    root = _object(doc, _NORM_BENCH_KEYS, "benchmark")
    if (root["schema_version"] != SCHEMA_VERSION or root["result"] != "pass"
            or root["operator"] != "rms_norm_f32"
            or root["model_shape"] != "SmolLM2-135M hidden_size=576"):
        raise SchemaError("benchmark: identity fields do not match")
    gpu = _object(root["gpu"], ("name", "compute_capability"), "benchmark.gpu")
    _text(gpu["name"], "gpu.name")
    _text(gpu["compute_capability"], "gpu.compute_capability")
    cells = root["measurements"]
    if type(cells) is not list or len(cells) != len(NORM_BENCH_ROWS):
        raise SchemaError("benchmark.measurements: expected 4 cases")
    for i, raw in enumerate(cells):
        where = f"measurements[{i}]"
        cell = _object(raw, _NORM_CELL_KEYS, where)
        if _int(cell["rows"], where + ".rows", 1) != NORM_BENCH_ROWS[i]:
            raise SchemaError(f"{where}: rows {cell['rows']} out of order")
        if cell["hidden_size"] != HEAD_BENCH_HIDDEN:
            raise SchemaError(f"{where}: hidden_size is not 576")
        _int(cell["iterations"], where + ".iterations", 1)
        for k in ("average_microseconds", "logical_gib_per_second"):
            _float(cell[k], f"{where}.{k}", positive=True)


def compare_with_l4(doc) -> List[dict]:
    """Per cell: this run's restricted and full times next to the reference's
    published L4 times, and the ratios (L4 time / this time)."""
    out = []
    for cell in doc["measurements"]:
        key = (cell["rows"], cell["allowed_tokens_per_row"])
        l4_full, l4_restricted = L4_OUTPUT_HEAD_US[key]
        out.append({
            "rows": key[0], "allowed": key[1],
            "restricted_us": cell["restricted_average_microseconds"],
            "full_us": cell["full_average_microseconds"],
            "l4_restricted_us": l4_restricted, "l4_full_us": l4_full,
            "restricted_vs_l4": round(l4_restricted / cell["restricted_average_microseconds"], 3),
            "full_vs_l4": round(l4_full / cell["full_average_microseconds"], 3),
        })
    return out


# ---- inference run contract -------------------------------------------------

_SHA1_HEX = re.compile(r"[0-9a-f]{40}")
_SHA256_HEX = re.compile(r"[0-9a-f]{64}")
_CAPABILITY = re.compile(r"(?:cpu|[0-9]+\.[0-9]+)")
BACKEND_MODES = ("cpu_reference", "eager", "cuda_graph", "ordinary")
DTYPES = ("float32", "float16", "bfloat16")
FINISH_REASONS = ("length", "eos", "stop")


@dataclass(frozen=True)
class RequestRecord:
    """One request of a run (contract.py:66-71)."""
    request_id: str
    prompt_token_ids: Tuple[int, ...]
    generated_token_ids: Tuple[int, ...]
    finish_reason: str


@dataclass(frozen=True)
class RunRecord:
    """An inference run in the contract's field layout (contract.py:85-160).
    ``to_json`` checks the document before it returns it."""
    commit: str
    bundle_sha256: str
    backend_name: str
    backend_version: str
    backend_mode: str
    model_id: str
    model_repository: str
    model_revision: str
    checkpoint_sha256: str
    vocabulary_size: int
    device_name: str
    compute_capability: str
    runtime_version: str
    dtype: str
    seed: int
    max_output_tokens: int
    requests: Tuple[RequestRecord, ...]
    model_load_seconds: float
    inference_seconds: float
    peak_gpu_memory_bytes: int
    temperature: float = 0.0
    prefix_caching: bool = False
    graphs: bool = False
    structured_output: bool = True

    def payload(self) -> dict:
        n_in = sum(len(r.prompt_token_ids) for r in self.requests)
        n_out = sum(len(r.generated_token_ids) for r in self.requests)
        doc = {
            "schema_version": SCHEMA_VERSION,
            "result": "pass",
            "source": {"commit": self.commit, "bundle_sha256": self.bundle_sha256},
            "backend": {"name": self.backend_name, "version": self.backend_version,
                        "mode": self.backend_mode},
            "model": {"id": self.model_id, "repository": self.model_repository,
                      "revision": self.model_revision,
                      "checkpoint_sha256": self.checkpoint_sha256,
                      "vocabulary_size": self.vocabulary_size},
            # the contract's field name is cuda_version; it carries the HIP
            # runtime version here
            "hardware": {"device_name": self.device_name,
                         "compute_capability": self.compute_capability,
                         "cuda_version": self.runtime_version},
            "generation": {"dtype": self.dtype, "temperature": float(self.temperature),
                           "seed": self.seed, "max_output_tokens": self.max_output_tokens},
            "features": {"prefix_caching": self.prefix_caching, "cuda_graphs": self.graphs,
                         "structured_output": self.structured_output},
            "requests": [{"request_id": r.request_id,
                          "prompt_token_ids": list(r.prompt_token_ids),
                          "generated_token_ids": list(r.generated_token_ids),
                          "finish_reason": r.finish_reason} for r in self.requests],
            "metrics": {
                "model_load_seconds": float(self.model_load_seconds),
                "inference_seconds": float(self.inference_seconds),
                "input_tokens": n_in,
                "output_tokens": n_out,
                "requests_per_second": len(self.requests) / self.inference_seconds,
                "output_tokens_per_second": n_out / self.inference_seconds,
                "peak_gpu_memory_bytes": int(self.peak_gpu_memory_bytes),
            },
        }
        check_run(doc)
        return doc

    def to_json(self) -> str:
        # compact, sorted, no NaN/Inf (contract.py:162-168)
        return json.dumps(self.payload(), allow_nan=False, sort_keys=True,
                          separators=(",", ":"))


_RUN_KEYS = ("schema_version", "result", "source", "backend", "model", "hardware",
             "generation", "features", "requests", "metrics")


def _token_list(value, where: str, vocab: int, allow_empty: bool) -> List[int]:
    if type(value) is not list or (not allow_empty and not value):
        raise SchemaError(f"{where}: expected a token list")
    for i, t in enumerate(value):
        if _int(t, f"{where}[{i}]") >= vocab:
            raise SchemaError(f"{where}[{i}]: token {t} is outside the vocabulary")
    return value


def check_run(doc) -> None:
    """Raises SchemaError unless ``doc`` satisfies the run contract
    (contract.py:229-428): exact field sets, identity formats, greedy
    generation, token ranges, and metrics consistent with the requests."""
    root = _object(doc, _RUN_KEYS, "run")
    if type(root["schema_version"]) is not int or root["schema_version"] != SCHEMA_VERSION \
            or root["result"] != "pass":
        raise SchemaError("run: schema_version or result")
    src = _object(root["source"], ("commit", "bundle_sha256"), "source")
    if not _SHA1_HEX.fullmatch(_text(src["commit"], "source.commit")):
        raise SchemaError("source.commit: expected a lowercase git object id")
    if not _SHA256_HEX.fullmatch(_text(src["bundle_sha256"], "source.bundle_sha256")):
        raise SchemaError("source.bundle_sha256: expected lowercase SHA-256")
    be = _object(root["backend"], ("name", "version", "mode"), "backend")
    _text(be["name"], "backend.name")
    _text(be["version"], "backend.version")
    if be["mode"] not in BACKEND_MODES:
        raise SchemaError("backend.mode: unsupported")
    model = _object(root["model"], ("id", "repository", "revision", "checkpoint_sha256",
                                    "vocabulary_size"), "model")
    _text(model["id"], "model.id")
    _text(model["repository"], "model.repository")
    if not _SHA1_HEX.fullmatch(_text(model["revision"], "model.revision")):
        raise SchemaError("model.revision: expected a lowercase commit")
    if not _SHA256_HEX.fullmatch(_text(model["checkpoint_sha256"], "model.checkpoint_sha256")):
        raise SchemaError("model.checkpoint_sha256: expected lowercase SHA-256")
    vocab = _int(model["vocabulary_size"], "model.vocabulary_size", 1)
    hw = _object(root["hardware"], ("device_name", "compute_capability", "cuda_version"),
                 "hardware")
    _text(hw["device_name"], "hardware.device_name")
    if not _CAPABILITY.fullmatch(_text(hw["compute_capability"], "hardware.compute_capability")):
        raise SchemaError("hardware.compute_capability: malformed")
    _text(hw["cuda_version"], "hardware.cuda_version")
    gen = _object(root["generation"], ("dtype", "temperature", "seed", "max_output_tokens"),
                  "generation")
    if gen["dtype"] not in DTYPES:
        raise SchemaError("generation.dtype: unsupported")
    if _float(gen["temperature"], "generation.temperature") != 0.0:
        raise SchemaError("generation.temperature: runs are greedy (0.0)")
    _int(gen["seed"], "generation.seed")
    cap = _int(gen["max_output_tokens"], "generation.max_output_tokens", 1)
    feats = _object(root["features"], ("prefix_caching", "cuda_graphs", "structured_output"),
                    "features")
    for k, v in feats.items():
        _flag(v, f"features.{k}")
    reqs = root["requests"]
    if type(reqs) is not list or not reqs:
        raise SchemaError("requests: expected a non-empty list")
    ids = set()
    n_in = n_out = 0
    for i, raw in enumerate(reqs):
        where = f"requests[{i}]"
        r = _object(raw, ("request_id", "prompt_token_ids", "generated_token_ids",
                          "finish_reason"), where)
        rid = _text(r["request_id"], where + ".request_id")
        if rid in ids:
            raise SchemaError(f"{where}: request id {rid!r} repeats")
        ids.add(rid)
        n_in += len(_token_list(r["prompt_token_ids"], where + ".prompt_token_ids", vocab, False))
        gen_tokens = _token_list(r["generated_token_ids"], where + ".generated_token_ids", vocab,
                                 True)
        if len(gen_tokens) > cap:
            raise SchemaError(f"{where}: more generated tokens than max_output_tokens")
        n_out += len(gen_tokens)
        if r["finish_reason"] not in FINISH_REASONS:
            raise SchemaError(f"{where}.finish_reason: unsupported")
    m = _object(root["metrics"], ("model_load_seconds", "inference_seconds", "input_tokens",
                                  "output_tokens", "requests_per_second",
                                  "output_tokens_per_second", "peak_gpu_memory_bytes"), "metrics")
    _float(m["model_load_seconds"], "metrics.model_load_seconds")
    t = _float(m["inference_seconds"], "metrics.inference_seconds", positive=True)
    if _int(m["input_tokens"], "metrics.input_tokens") != n_in:
        raise SchemaError("metrics.input_tokens: does not match the requests")
    if _int(m["output_tokens"], "metrics.output_tokens") != n_out:
        raise SchemaError("metrics.output_tokens: does not match the requests")
    rps = _float(m["requests_per_second"], "metrics.requests_per_second", positive=True)
    tps = _float(m["output_tokens_per_second"], "metrics.output_tokens_per_second")
    _int(m["peak_gpu_memory_bytes"], "metrics.peak_gpu_memory_bytes")
    if not math.isclose(rps, len(reqs) / t, rel_tol=1e-9):
        raise SchemaError("metrics.requests_per_second: inconsistent with the run")
    if not math.isclose(tps, n_out / t, rel_tol=1e-9):
        raise SchemaError("metrics.output_tokens_per_second: inconsistent with the run")


def load_run(text: str) -> dict:
    """Parses a run document strictly (duplicate keys and NaN/Infinity are
    errors, contract.py:429-448) and checks it."""
    def no_duplicates(pairs: Sequence[Tuple[str, object]]) -> dict:
        out = {}
        for k, v in pairs:
            if k in out:
                raise SchemaError(f"duplicate JSON key {k!r}")
            out[k] = v
        return out

    def no_constants(name: str):
        raise SchemaError(f"non-finite JSON constant {name}")

    doc = json.loads(text, object_pairs_hook=no_duplicates, parse_constant=no_constants)
    check_run(doc)
    return doc
