"""The reference result schemas (market_sim_amd/schema.py): the run contract
(tools/inference/contract.py) restated with the reference's own test cases
(tools/inference/test_contract.py:19-122), and the output-head benchmark
document (tools/modal/vllm_modal_app.py:459-516)."""
import copy
import json

import pytest

from market_sim_amd import schema


def _valid_run() -> schema.RunRecord:
    # the reference's valid_run() (test_contract.py:19-43)
    return schema.RunRecord(
        commit="c" * 40, bundle_sha256="d" * 64,
        backend_name="vllm", backend_version="0.25.1", backend_mode="eager",
        model_id="smollm2-135m", model_repository="HuggingFaceTB/SmolLM2-135M",
        model_revision="a" * 40, checkpoint_sha256="b" * 64, vocabulary_size=49_152,
        device_name="NVIDIA L4", compute_capability="8.9", runtime_version="12.9",
        dtype="float16", seed=0, max_output_tokens=3,
        requests=(schema.RequestRecord("pr4-greedy", (0, 1, 2, 3), (198, 198, 504), "length"),),
        model_load_seconds=1.0, inference_seconds=0.5, peak_gpu_memory_bytes=1_024,
        prefix_caching=False, graphs=False, structured_output=False)


def test_run_payload_has_the_contract_layout():
    # contract.py:100-160, written out field by field
    expected = {
        "schema_version": 1, "result": "pass",
        "source": {"commit": "c" * 40, "bundle_sha256": "d" * 64},
        "backend": {"name": "vllm", "version": "0.25.1", "mode": "eager"},
        "model": {"id": "smollm2-135m", "repository": "HuggingFaceTB/SmolLM2-135M",
                  "revision": "a" * 40, "checkpoint_sha256": "b" * 64,
                  "vocabulary_size": 49152},
        "hardware": {"device_name": "NVIDIA L4", "compute_capability": "8.9",
                     "cuda_version": "12.9"},
        "generation": {"dtype": "float16", "temperature": 0.0, "seed": 0,
                       "max_output_tokens": 3},
        "features": {"prefix_caching": False, "cuda_graphs": False,
                     "structured_output": False},
        "requests": [{"request_id": "pr4-greedy", "prompt_token_ids": [0, 1, 2, 3],
                      "generated_token_ids": [198, 198, 504], "finish_reason": "length"}],
        # RunMetrics(1.0, 0.5, 4, 3, 2.0, 6.0, 1_024) of the reference test
        "metrics": {"model_load_seconds": 1.0, "inference_seconds": 0.5, "input_tokens": 4,
                    "output_tokens": 3, "requests_per_second": 2.0,
                    "output_tokens_per_second": 6.0, "peak_gpu_memory_bytes": 1024},
    }
    assert _valid_run().payload() == expected


def test_round_trip_is_strict_and_deterministic():
    run = _valid_run()
    text = run.to_json()
    assert schema.load_run(text) == run.payload()
    assert text == run.to_json()
    assert text == json.dumps(json.loads(text), sort_keys=True, separators=(",", ":"))


@pytest.mark.parametrize("text", ['{"schema_version":1,"schema_version":1}', '{"value":NaN}'])
def test_rejects_duplicate_and_non_finite_json(text):
    with pytest.raises(schema.SchemaError):
        schema.load_run(text)


@pytest.mark.parametrize("path,value", [
    (("schema_version",), True), (("result",), "failure"),
    (("source", "commit"), "dirty"), (("source", "bundle_sha256"), "short"),
    (("backend", "mode"), "unknown"), (("model", "revision"), "moving-main"),
    (("model", "checkpoint_sha256"), "short"), (("hardware", "compute_capability"), "L4"),
    (("generation", "temperature"), 0.1), (("features", "cuda_graphs"), 1),
    (("metrics", "input_tokens"), 5), (("metrics", "requests_per_second"), 3.0),
])
def test_rejects_schema_and_provenance_mutations(path, value):
    doc = _valid_run().payload()
    target = doc
    for k in path[:-1]:
        target = target[k]
    target[path[-1]] = value
    with pytest.raises(schema.SchemaError):
        schema.check_run(doc)


@pytest.mark.parametrize("field,value", [
    ("request_id", None), ("prompt_token_ids", [49_152]),
    ("generated_token_ids", [1, 2, 3, 4]), ("finish_reason", "cancelled"),
])
def test_rejects_token_and_request_inconsistency(field, value):
    doc = _valid_run().payload()
    if field == "request_id":
        doc["requests"].append(copy.deepcopy(doc["requests"][0]))
    else:
        doc["requests"][0][field] = value
    with pytest.raises(schema.SchemaError):
        schema.check_run(doc)


def test_mi355x_identity_is_accepted():
    run = _valid_run()
    doc = run.payload()
    doc["hardware"] = {"device_name": "AMD gfx950", "compute_capability": "9.5",
                       "cuda_version": "7.2.0"}
    schema.check_run(doc)


def _head_doc():
    cells = []
    for rows in schema.HEAD_BENCH_ROWS:
        for allowed in schema.HEAD_BENCH_ALLOWED:
            cells.append({
                "rows": rows, "allowed_tokens_per_row": allowed, "iterations": 100,
                "full_average_microseconds": 20.0, "restricted_average_microseconds": 5.0,
                "speedup": 4.0, "full_scores": rows * 49152, "restricted_scores": rows * allowed,
                "materialized_logit_bytes_avoided": rows * 49152 * 2,
                "exact_token_parity": True})
    return {"schema_version": 1, "result": "pass", "operator": "restricted_output_head_f16",
            "model_shape": "SmolLM2-135M", "hidden_size": 576, "vocabulary_size": 49152,
            "gpu": {"name": "AMD gfx950", "compute_capability": "9.5"}, "measurements": cells}


def test_output_head_benchmark_document():
    doc = _head_doc()
    schema.check_output_head_benchmark(doc, "gfx950", "9.5")
    cmp = schema.compare_with_l4(doc)
    assert len(cmp) == 12 and cmp[0]["l4_restricted_us"] == 12.872
    assert cmp[-1]["restricted_vs_l4"] == round(294.144 / 5.0, 3)


@pytest.mark.parametrize("mutate", [
    lambda d: d.pop("gpu"),
    lambda d: d.__setitem__("hidden_size", 2048),
    lambda d: d["gpu"].__setitem__("compute_capability", "8.9"),
    lambda d: d["measurements"].pop(),
    lambda d: d["measurements"].__setitem__(1, copy.deepcopy(d["measurements"][0])),
    lambda d: d["measurements"][3].__setitem__("exact_token_parity", False),
    lambda d: d["measurements"][5].__setitem__("restricted_scores", 1),
    lambda d: d["measurements"][7].__setitem__("speedup", 2),
    lambda d: d["measurements"][9].__setitem__("full_average_microseconds", float("inf")),
])
def test_output_head_benchmark_rejects_mutations(mutate):
    doc = _head_doc()
    mutate(doc)
    with pytest.raises(schema.SchemaError):
        schema.check_output_head_benchmark(doc, "gfx950", "9.5")


def _greedy_doc():
    return {"schema_version": 1, "result": "pass", "operator": "restricted_greedy_f16",
            "grammar": "smollm2_market_action_v1", "vocabulary_size": 49152,
            "grammar_states": 3230, "grammar_arcs": 3229, "maximum_allowed_tokens": 11,
            "gpu": {"name": "AMD gfx950", "compute_capability": "9.5"},
            "measurements": [{"rows": r, "total_allowed_candidates": 3 * r, "iterations": 10,
                              "average_microseconds": 9.5, "sequences_per_second": 1e5,
                              "candidate_gib_per_second": 0.01} for r in (1, 16, 256)]}


def _norm_doc():
    return {"schema_version": 1, "result": "pass", "operator": "rms_norm_f32",
            "model_shape": "SmolLM2-135M hidden_size=576",
            "gpu": {"name": "AMD gfx950", "compute_capability": "9.5"},
            "measurements": [{"rows": r, "hidden_size": 576, "iterations": 10,
                              "average_microseconds": 4.0, "logical_gib_per_second": 1.5}
                             for r in (1, 16, 256, 1024)]}


def test_secondary_benchmark_documents_accepted_and_rejected():
    """The reference validator's rules (vllm_modal_app.py:283-427): exactly
    the reference fields, the fixed identity, the case order, positive
    finite rates."""
    schema.check_restricted_greedy_benchmark(_greedy_doc())
    schema.check_rmsnorm_benchmark(_norm_doc())
    bad = []
    d = _greedy_doc(); d["measurements"][0]["token_parity"] = True; bad.append((schema.check_restricted_greedy_benchmark, d))
    d = _greedy_doc(); d["grammar"] = "other"; bad.append((schema.check_restricted_greedy_benchmark, d))
    d = _greedy_doc(); d["measurements"][2]["candidate_gib_per_second"] = 0.0; bad.append((schema.check_restricted_greedy_benchmark, d))
    d = _greedy_doc(); d["measurements"] = d["measurements"][::-1]; bad.append((schema.check_restricted_greedy_benchmark, d))
    d = _norm_doc(); del d["measurements"][1]["iterations"]; bad.append((schema.check_rmsnorm_benchmark, d))
    d = _norm_doc(); d["measurements"][0]["hidden_size"] = 2048; bad.append((schema.check_rmsnorm_benchmark, d))
    d = _norm_doc(); d["measurements"][3]["average_microseconds"] = float("inf"); bad.append((schema.check_rmsnorm_benchmark, d))
    d = _norm_doc(); d["operator"] = "rms_norm_f16"; bad.append((schema.check_rmsnorm_benchmark, d))
    for fn, doc in bad:
        with pytest.raises(schema.SchemaError):
            fn(doc)
