"""The C++ caller of the C ABI (ghost-infer_amd/gi_layer_harness): one layer's attention played as the
reference's layer loop plays it (layer_attn src/cuda.rs:9706-9717, GpuModel::attention
src/cuda.rs:8448-8541): a prompt through the cache write and the prefill path, then decode steps replayed
from one captured HIP graph with a device-side position, every output row checked inside the harness
against the exact split path over the whole sequence."""
import json
import os
import subprocess
import sys

import pytest

HARNESS = os.path.join(os.path.dirname(os.path.abspath(__file__)), "..", "ghost-infer_amd", "gi_layer_harness")


@pytest.mark.gpu
@pytest.mark.parametrize("args", [[], ["--int8"], ["--heads", "16", "--kv", "2", "--hd", "256", "--prompt", "100",
                                                   "--steps", "10"], ["--no-graph", "--prompt", "40", "--steps", "6",
                                                                      "--heads", "32", "--kv", "4"]])
def test_layer_harness(args):
    assert os.path.exists(HARNESS), "gi_layer_harness is not built (run __graft_entry__.build())"
    print("harness", " ".join(args), flush=True)
    r = subprocess.run([HARNESS, *args], capture_output=True, text=True, timeout=120)
    sys.stdout.write(r.stdout)
    sys.stderr.write(r.stderr)
    assert r.returncode == 0, f"harness exit {r.returncode}: {r.stderr.strip() or r.stdout.strip()}"
    line = json.loads(r.stdout.strip().splitlines()[-1])
    assert line["ok"] and line["max_abs_decode"] <= line["tol_decode"] and line["max_abs_prompt"] <= line["tol_prompt"]
