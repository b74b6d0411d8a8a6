"""The bench's compact JSON line: per-launch tables, agreement columns, section order (CPU only)."""

import importlib.util
import json
import os

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", os.path.join(ROOT, "bench.py"))
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)
    return module


def _agreement(ulp):
    return {"max_abs": 1e-3 * ulp, "max_ulp": float(ulp), "flips": ulp, "over_2e-3": 0, "rel_l2": 1e-6, "count": 64}


def _result():
    launches = {f"{p}_m{m}": {"us": 10.0 * (i + 1) + m, "GB/s": 1000.0 + m, "route": "venturi-q8-mfma"}
                for i, p in enumerate(("qkv", "o_proj", "gate_up", "down")) for m in (1, 4, 8, 16)}
    a8 = {f"{p}_m{m}_p{passes}": {"us": 5.0 + m + passes, "GB/s": 900.0}
          for passes in (1, 2) for p in ("qkv", "down") for m in (1, 8)}
    return {
        "metric": "m", "value": 1.0, "unit": "GB/s", "n_gpus": 1, "steps": 2, "warmup": 1, "ms_per_step": 0.3,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp16", "data": "synthetic",
        "config": {"workload": "w"}, "roofline": {"frac": 0.6},
        "parity": {"summary": _agreement(12), "per_launch": {k: _agreement(3) for k in launches}},
        "per_launch": launches,
        "exact_route": {"per_launch": {k: {"us": 20.0, "GB/s": 500.0} for k in launches}},
        "a8_decode": {"GB/s": 3900.0, "per_launch": a8},
        "vocab_head": {"per_launch": {"m1": {"us": 205.0}, "m1_exact_route": {"us": 255.0}}},
        "prefill_a8": {"parity": {"summary": _agreement(54), "per_projection": {"qkv": _agreement(15)}},
                       "stages": {"qkv": {"us": 475.2, "TOPS": 316.3, "frac_int8_peak": 0.06}},
                       "cpu_baseline": {"value": 1.0, "unit": "TOP/s", "cores": 16, "kind": "oracle", "sample": "s"}},
        "prefill_a16": {"w4a16": {"TFLOP/s": 1100.0, "library_route": {"kernel": "k", "TFLOP/s": 1100.0, "note": "n",
                                                                       "parity": _agreement(43)},
                                  "stages": {"qkv": {"us": 123.0, "TFLOP/s": 1200.0, "fused_mfma_us": 150.0}}}},
        "q56_decode": {"q5": {"GB/s": 3100.0, "roofline": {"frac": 0.39},
                              "per_launch": {f"qkv_m{m}": {"us": 9.0, "GB/s": 2000.0} for m in (1, 4)}}},
        "cpu_baseline": {"value": 12.0},
    }


def test_launch_table_groups_by_projection_and_pass():
    bench = _bench()
    table = bench.launch_table(_result()["a8_decode"]["per_launch"])
    assert table["M"] == [1, 8]
    assert table["us"]["qkv_p1"] == [7.0, 14.0] and table["us"]["down_p2"] == [8.0, 15.0]
    assert table["GB/s"]["qkv_p2"] == [900.0, 900.0]


def test_launch_table_leaves_other_keys_alone():
    bench = _bench()
    records = _result()["vocab_head"]["per_launch"]
    assert bench.launch_table(records) == records


def test_shorten_keeps_sections_and_orders_them():
    bench = _bench()
    full = _result()
    short = bench.shorten(full)
    assert set(short) == set(full)
    keys = list(short)
    assert keys[:2] == ["metric", "value"] and keys[-3:] == ["exact_route", "parity", "per_launch"]
    # Headline launches keep both columns and the uniform route once.
    assert short["per_launch"]["us"]["gate_up"] == [31.0, 34.0, 38.0, 46.0]
    assert short["per_launch"]["GB/s"]["qkv"] == [1001.0, 1004.0, 1008.0, 1016.0]
    assert short["per_launch"]["route"] == "venturi-q8-mfma"
    assert "GB/s" in short["exact_route"]["per_launch"]
    # Elsewhere the rate columns go (the section keeps its own GB/s).
    assert "GB/s" not in short["a8_decode"]["per_launch"] and short["a8_decode"]["GB/s"] == 3900.0
    # Agreement records: the summary stays whole, per-launch keeps max-ulp arrays.
    assert short["parity"]["summary"] == full["parity"]["summary"]
    assert short["parity"]["per_launch"]["max_ulp"]["down"] == [3.0, 3.0, 3.0, 3.0]
    assert "per_projection" not in short["prefill_a8"]["parity"]
    assert short["prefill_a8"]["stages"]["qkv"] == {"us": 475.2, "TOPS": 316.3}
    # Prefill stages keep their times, the library route its rate, Q5/Q6 their section rates;
    # section baselines drop the sample text (the headline's keeps it).
    w4 = short["prefill_a16"]["w4a16"]
    assert w4["stages"]["qkv"] == {"us": 123.0, "fused_mfma_us": 150.0}
    assert w4["library_route"] == {"kernel": "k", "TFLOP/s": 1100.0}
    assert short["q56_decode"]["q5"] == {"GB/s": 3100.0, "roofline": {"frac": 0.39}}
    assert "sample" not in short["prefill_a8"]["cpu_baseline"] and short["prefill_a8"]["cpu_baseline"]["value"] == 1.0
    assert short["cpu_baseline"] == full["cpu_baseline"]
    json.dumps(short)  # still one JSON object
