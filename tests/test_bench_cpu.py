"""CPU checks of bench.py's roofline bookkeeping (no GPU, no kernel calls)."""
import importlib.util
import os

import pytest

from market_sim_amd import workloads

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _fracs(d):
    """Every value of a key ending in 'frac' or 'util', nested."""
    out = []
    for k, v in d.items():
        if isinstance(v, dict):
            out += _fracs(v)
        elif k.endswith("frac") or k.endswith("util"):
            out.append(v)
    return out


def test_fallback_summary_without_unrestricted_rows_has_no_fraction():
    bench = _bench()
    w = workloads.config(4, seed=0, scale_vocab=2048, scale_rows=16)
    alg = bench.algorithmic_bytes(w)
    assert alg["B_u"] == 0
    # an empty unrestricted stage still takes a few microseconds to launch:
    # the head's bytes over that time would read as a fraction far above 1
    for fb_ms in (None, 0.004):
        fb = bench.fallback_summary(alg, fb_ms)
        assert fb == {"kernel": "none (no unrestricted rows)", "rows": 0}
        assert all(f <= 1.0 for f in _fracs(fb))


def test_fallback_summary_with_unrestricted_rows():
    bench = _bench()
    w = workloads.config(3, seed=0, scale_vocab=4096, scale_rows=64)
    alg = bench.algorithmic_bytes(w)
    assert alg["B_u"] > 0
    # a head launch moving its bytes at half of the HBM peak
    fb_ms = alg["fallback_bytes"] / (0.5 * bench.HBM_PEAK_GBS * 1e9) * 1e3
    fb = bench.fallback_summary(alg, fb_ms)
    assert fb["rows"] == alg["B_u"]
    assert fb["hbm_frac"] == pytest.approx(0.5, abs=1e-3)
    assert all(0.0 <= f <= 1.0 for f in _fracs(fb))


def test_profiled_traffic_reads_only_the_workloads_own_summary(tmp_path, monkeypatch):
    bench = _bench()
    monkeypatch.setattr(bench, "ROOT", str(tmp_path))
    (tmp_path / "profiles").mkdir()
    (tmp_path / "profiles" / "decode_tail_cfg2_traffic.md").write_text(
        "# t\n\ntraffic_bytes_per_launch pass_kernel<18> = 1234\n")
    assert bench.profiled_traffic("pass_kernel", "cfg2") == (
        1234, os.path.join("profiles", "decode_tail_cfg2_traffic.md"))
    # another workload's figure is never borrowed
    assert bench.profiled_traffic("pass_kernel", "cfg3") == (None, None)
    assert bench.profiled_traffic("gather_mfma_kernel", "cfg2") == (None, None)


def test_algorithmic_pass_bytes_count_the_table_once_with_unrestricted_rows():
    bench = _bench()
    w = workloads.config(3, seed=0, scale_vocab=4096, scale_rows=64)
    alg = bench.algorithmic_bytes(w)
    H, V, B = w.hidden, w.vocab, w.rows
    assert alg["pass_bytes"] == (2 * H * V + 4 * alg["N"] + 4 * H * B + 4 * (alg["B_r"] + 1)
                                 + 12 * B)


def test_cpu_baseline_on_the_pre_decoded_table_gives_the_same_bits():
    """cpu_baseline times the oracle on the FP16 table decoded to FP32 before
    the timed region; its outputs (the parity leg's expected values) must be
    the bits the FP16 table gives."""
    import numpy as np

    import oracle
    bench = _bench()
    w = workloads.config(3, seed=4, scale_vocab=3000, scale_rows=24)
    cb = bench.cpu_baseline(w, 0.05)
    tok, sc, nx = cb.pop("_outputs")
    etok, esc, enx = oracle.decode_tail(w.x, w.norm_weight, w.epsilon, w.embedding,
                                        w.row_state, w.state_offsets, w.state_tokens, threads=4)
    assert np.array_equal(tok, etok) and np.array_equal(nx, enx)
    assert np.array_equal(sc.view(np.uint32), esc.view(np.uint32))
    assert cb["kind"] == "port" and cb["cores"] >= 1 and "pre-decoded" in cb["sample"]
