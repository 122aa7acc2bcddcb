"""The bench's printed line: every benchmark config's figures fit in a record that keeps only the output's end."""
import json
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def _roof(bound, v, peak, unit):
    return {"bound": bound, "achieved": v, "peak": peak, "unit": unit, "frac": round(v / peak, 4),
            "traffic": 123456789, "kernel": "gi_something_long_kernel_name (split-K pass)",
            "algorithmic_bytes_per_launch": 134234112, "kernel_ms_per_launch": 0.023241, "launches_timed": 200,
            "combine_ms_per_launch": 0.004512, "step_frac_of_hbm_peak": 0.6525}


def _entry(v, unit, peak, bound, cfg=None):
    return {"value": v, "unit": unit, "ms_per_step": 0.0257112503, "dtype": "f16 K/V, f32 math",
            "config": cfg or {"workload": "x" * 90, "ctx": 65536}, "roofline": _roof(bound, v * 1.1, peak, unit)}


def full_result():
    """A record shaped like the default run's, with the longest field values the bench writes."""
    r = {"metric": bench.METRIC, "n_gpus": 1, "steps": 200, "warmup": 20, "higher_is_better": True,
         "scaling": "weak", "vs_baseline": None, "data": "synthetic"}
    r.update(_entry(5555.5, "GB/s", 8000.0, "hbm",
                    {"workload": "config 2: decode, 1 token, ctx 65536, 32q/4kv, hd 128", "ctx": 65536,
                     "n_tok": 1, "n_heads": 32, "n_kv": 4, "hd": 128, "kv_bytes_per_step": 134217728,
                     "layers_rotated": 4, "slices": 64, "keys_per_slice": 1024, "kv_layout": "head_major"}))
    sec = {w: _entry(2222.2, "GB/s", 8000.0, "hbm") for w in ("decode4k", "verify")}
    sec["prefill8k"] = _entry(1111.1, "TFLOP/s", 2500.0, "mfma")
    sec["chunked"] = _entry(1111.1, "TFLOP/s", 2500.0, "mfma",
                            {"workload": "config 5", "total_seconds": 0.1324532579, "total_flops": 140738562097152,
                             "per_chunk_tflops": [1111.1] * 64})
    for w in ("decode64k_i8", "verify_i8", "decode64k_h256", "verify_h256", "decode64k_h256_i8", "verify_h256_i8",
              "decode64k_h256_q4", "verify_h256_q4", "decode64k_h64", "verify_h64"):
        sec[w] = _entry(2222.2, "GB/s", 8000.0, "hbm")
    for w in ("prefill8k_i8", "prefill8k_h256", "prefill8k_h256_i8", "prefill8k_h256_q4", "prefill8k_h64"):
        sec[w] = _entry(1111.1, "TFLOP/s", 2500.0, "mfma")
    sec["hbm_copy_measured_GBs"] = 5072.2
    sec["peaks_measured"] = {"mfma_f16_dense_TFLOPs": 2171.9, "mfma_f16_dense_random_operands_TFLOPs": 1651.7,
                             "hbm_read_GBs_1GiB": 6965.9, "hbm_read_GBs_134MB": 6017.6}
    r["secondary"] = sec
    r["cpu_baseline"] = {"value": 6.851, "unit": "GB/s", "cores": 16, "kind": "port", "sample": "y" * 400,
                         "sample_short": "decode64k: 200 runs, oracle Model::attention, f32 cache",
                         "runs": [{"config": "decode64k", "value": 1.0}] * 6}
    return r


def test_compact_line_fits_and_holds_every_config():
    line = json.dumps(bench.compact_line(full_result()), separators=(",", ":"))
    assert len(line) < 2200, len(line)
    d = json.loads(line)
    for k in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
              "scaling", "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline"):
        assert k in d, k
    for k in ("bound", "achieved", "peak", "unit", "frac", "traffic"):
        assert k in d["roofline"]
    for w in ("decode4k", "verify", "prefill8k", "chunked"):
        e = d["secondary"][w]
        assert {"value", "unit", "ms_per_step", "roofline"} <= set(e)
        assert e["roofline"]["frac"] > 0
    assert "total_s" in d["secondary"]["chunked"]
    assert len(d["secondary"]["chunked"]["per_chunk_tflops_every16"]) == 5
    assert "verify_h256_q4=" in d["secondary"]["frac_other"]
    assert d["cpu_baseline"]["cores"] == 16 and d["cpu_baseline"]["kind"] == "port"
