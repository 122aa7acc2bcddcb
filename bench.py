"""Benchmark of the gfx950 attention hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload decode64k|decode4k|verify|prefill8k|chunked|qkrope|
                    decode64k_i8|verify_i8|prefill8k_i8|decode64k_h256|verify_h256|prefill8k_h256|
                    decode64k_h256_i8|verify_h256_i8|prefill8k_h256_i8|decode64k_h256_q4|verify_h256_q4|
                    prefill8k_h256_q4|decode64k_h64|decode64k_h64_i8|prefill8k_h64|prefill8k_h64_i8|decode16k_h80|prefill8k_h96|
                    decode16k_h80_i8|prefill8k_h96_i8|prefill8k_f32]
                    [--no-cpu-baseline] [--no-secondary] [--reference-layout] [--verbose]
                    [--detail-out FILE] [--full-line]

A step is one pass of the hot path over one batch of synthetic seeded input already resident in HBM:
  decode64k  config 2: one token, 32 query / 4 kv heads, head 128, 65536-key f16 cache (the default: the
             headline metric's decode half, HBM GB/s of K+V bytes)
  decode4k   config 1: one token, 32 / 8 heads, 4096 keys
  verify     config 4: 8 draft tokens on a 32768-key prefix, 32 / 4 heads
  prefill8k  config 3: causal prefill of 8192 tokens, 32 / 8 heads, f16 in and out (MFMA TFLOP/s)
  chunked    config 5: 131072 tokens in 2048-token chunks against the growing cache, 32 / 4 heads
  qkrope     the cache write before attention (qk_norm_rope + f16 KV store) for config 3's 8192 tokens
  decode64k_h256, verify_h256, prefill8k_h256
             head size 256 (Qwen3.5-style 16 query / 2 kv heads): decode at 65536 keys, an 8-token verify at
             32768, prefill of 8192
  decode64k_h256_i8, verify_h256_i8, prefill8k_h256_i8
             head size 256 over the int8 cache (the reference's attention_decode_tc256 / prefill_tc256 shapes)
  decode64k_h256_q4, verify_h256_q4, prefill8k_h256_q4
             head size 256 over the 4-bit cache (the reference's --kv q4: 128 bytes a row plus 8 f16 scales)
  decode64k_h64, decode64k_h64_i8, prefill8k_h64, prefill8k_h64_i8
             head size 64 (Llama-3.2-1B-style 32 query / 8 kv heads) over the f16 and int8 caches
  decode16k_h80, prefill8k_h96, decode16k_h80_i8, prefill8k_h96_i8
             the f32 kernels' head sizes (Phi-2-style 80, Phi-3-style 96; 32 query / 32 kv heads), over the f16
             and int8 caches
  prefill8k_f32
             config 3's prompt in f32 (the reference's attention_prefill, GHOST_INFER_NO_TC_ATT)
  decode64k_i8, verify_i8, prefill8k_i8
             configs 2, 4 and 3 over the int8 cache (the reference's KV8 format: int8 rows, an f32 scale per
             position and kv head); bytes are the int8 rows plus their scales
Decode steps rotate over several layers' caches whose total exceeds the 256 MB Infinity Cache, as a
model's layer loop does, so no step finds its K/V in the last-level cache.

Prints ONE JSON line (rank 0), kept under ~2 KB so that a record holding only the end of the output holds
all of it. With the default workload the line also carries configs 1, 3, 4 and 5 under "secondary" (decode4k,
verify, prefill8k and chunked: value, time, roofline; chunked also the total time and every 16th chunk's
TFLOP/s) and the roofline fraction of every int8, head-64, head-256 and 4-bit workload; and the CPU baseline: the
oracle's restatement of the reference's CPU attention (src/model.rs:1320-1409) over the same inputs with the
cache widened to f32 (as the reference's CPU session holds it), timed on this host at its CPU share (up to 16
threads) and at half of it (the reference's default logical/2), for configs 2 and 1 and a bounded sample of
config 3. The full record (every field of every workload, every chunk, the box's measured peaks) goes to the
file --detail-out names; --full-line prints it instead. Progress messages go to
stderr with --verbose.
"""
import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "ghost-infer_amd"))

HBM_PEAK_GBS = 8000.0      # MI355X HBM3E, published
F16_DENSE_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 MFMA, published
FP32_DENSE_PEAK_TFLOPS = 157.3  # MI355X dense fp32 MFMA, published (the f32 kernels' prefill)
METRIC = "decode-attn HBM GB/s @64K ctx; prefill-attn TFLOPS @8K; % of roofline"
HD = 128


VERBOSE = bool(os.environ.get("GI_BENCH_VERBOSE"))


def log(*a):
    """Progress messages, on stderr only when asked for (--verbose or GI_BENCH_VERBOSE=1): a record that keeps
    the end of the output must find the result line there, not the progress."""
    if VERBOSE:
        print(*a, file=sys.stderr, flush=True)


def seeded_cache(gen, rows, n_kv, dev, torch, layout="reference", i8=False, hd=HD):
    """K and V caches of N(0,1) f16 values: [rows, n_kv, HD] (the reference's layout) or [n_kv, rows, HD]
    (head-major, each kv head's rows contiguous). i8: int8 rows round(40 N(0,1)) clipped to -127..127 and
    f32 scales in [0.02, 0.03] ([rows, n_kv] or [n_kv, rows]), like quantised N(0,1) rows. i8 == "q4": the
    4-bit cache (head size 256), random nibbles 1..15 in rows of 128 bytes and f16 scales in [0.2, 0.35], 8 a
    row. Returns (k, v, k_scale, v_scale)."""
    shape = (rows, n_kv, hd) if layout == "reference" else (n_kv, rows, hd)
    if i8 == "q4":
        def nib():
            return torch.randint(0, 256, shape[:2] + (128,), generator=gen, device=dev, dtype=torch.int32).to(
                torch.uint8) | 0x11

        def scl():
            return (torch.rand(shape[:2] + (8,), generator=gen, device=dev) * 0.15 + 0.2).half()

        return nib(), nib(), scl(), scl()
    if i8:
        def ints():
            x = torch.randn(shape, generator=gen, device=dev, dtype=torch.float32) * 40
            return x.round().clamp(-127, 127).to(torch.int8)

        k, v = ints(), ints()
        sc = shape[:2]
        ks = torch.rand(sc, generator=gen, device=dev, dtype=torch.float32) * 0.01 + 0.02
        vs = torch.rand(sc, generator=gen, device=dev, dtype=torch.float32) * 0.01 + 0.02
        return k, v, ks, vs
    k = torch.randn(shape, generator=gen, device=dev, dtype=torch.float32).half()
    v = torch.randn(shape, generator=gen, device=dev, dtype=torch.float32).half()
    return k, v, None, None


def kernel_times(gi_attn, fn, steps, torch, kinds, warm_steps=0):
    """Runs `steps` more steps eagerly with the library's per-kernel event timing on (HIP events recorded
    around each launch, on the stream it is launched on) and returns {kind: (mean ms per launch,
    launches)}. warm_steps untimed steps run first, right before them (the clocks drop during the spin
    below, and an MFMA-bound kernel of a few launches would otherwise be timed while they climb back)."""
    for k in kinds:
        gi_attn.kernel_timing_read(k)  # drop anything recorded before
    try:
        # a spin kernel in front keeps the GPU busy while the host enqueues every step, so each event pair
        # brackets its kernel back to back and not the host's submission gaps
        torch.cuda._sleep(int(5e7))
        for i in range(warm_steps):
            fn(i)
        gi_attn.kernel_timing(True)
        for i in range(steps):
            fn(i)
        torch.cuda.synchronize()
    finally:
        gi_attn.kernel_timing(False)
    res = {}
    for k in kinds:
        ms, n = gi_attn.kernel_timing_read(k)
        res[k] = (ms / n if n else None, n)
    return res


def decode_kernel_name(n_tok, n_heads, n_kv, hd, i8, chunk=None):
    """Name of the split-K kernel a decode call of this shape launches: the host library's variant rule
    (up to 8 (token, head) pairs per kv head: one column block with two columns per pair; above, one pair
    per MFMA column, with two column blocks per wave above 16 pairs at head size 128 (f16 above 32 pairs:
    two pair sets per workgroup, each over two waves), and two pair sets of one column block at head size
    256 over the f16 cache; over its int8 and 4-bit caches one pair per column throughout, 16 pairs per workgroup
    or, above 16 pairs, two pair sets (int8) or two column blocks per wave (4-bit)). The f16 head-128 kernel with up
    to 8 pairs has a short-span form (`..._1s`) for slices (`chunk` keys) of at most two tiles per wave."""
    pairs, p = n_tok * (n_heads // n_kv), 8
    if hd not in (64, 128, 256):  # the f32 kernels' head sizes
        return "gi_decode_f32" + ("_i8" if i8 else "") + f"_h{hd}"
    if hd == 256 and i8:  # the reference's tc256 roundings, one pair per column: 16 or 32 pairs per workgroup
        if pairs <= 2 * p:
            short = "s" if chunk is not None and chunk <= 128 else ""
            return "gi_decode_pm_1" + short + ("_q4" if i8 == "q4" else "_i8_h256")
        return "gi_decode_pm_2_q4" if i8 == "q4" else "gi_decode_pm_ws2_1_i8_h256"
    if pairs <= p:
        name = "gi_decode_partial_1"
        if chunk is not None and chunk <= (128 if hd == 256 else 512 if i8 else 256):
            return name + "s" + ("_i8" if i8 else "_h64" if hd == 64 else "_h256" if hd == 256 else "")
    elif hd == 64:
        name = "gi_decode_pm_2" if pairs > 2 * p else "gi_decode_pm_1"
    elif hd == 256:
        name = "gi_decode_pm_ws2_1"
    else:
        name = ("gi_decode_pm_ws2_2" if pairs > 4 * p and not i8 else
                "gi_decode_pm_2" if pairs > 2 * p else "gi_decode_pm_1")
    return name + ("_i8" if i8 else "") + ("_h256" if hd == 256 else "_h64" if hd == 64 else "")


def profile_traffic(name):
    """HBM bytes per launch of a kernel from the committed rocprofv3 --pmc summary profiles/<name>.md
    (its line "traffic_bytes_per_launch: N"), or None when there is none."""
    path = os.path.join(ROOT, "profiles", name + ".md")
    try:
        with open(path) as f:
            for line in f:
                if line.strip().startswith("traffic_bytes_per_launch:"):
                    return int(float(line.split(":", 1)[1]))
    except OSError:
        pass
    return None


# Seconds of untimed work before each timed region (besides the `warmup` steps): the GPU's clocks climb for
# tens of milliseconds after an idle spell, so a region that starts cold times the ramp (config 3's prefill
# measured 0.58 ms per launch over 20 launches and 0.52 ms over 200, on one box).
WARM_SECONDS = float(os.environ.get("GI_BENCH_WARM_SECONDS", "0.3"))


def warm_up(fn, warmup, torch):
    """Runs `warmup` untimed steps, and more until WARM_SECONDS of GPU time have passed."""
    t0 = time.perf_counter()
    i = 0
    while i < warmup or time.perf_counter() - t0 < WARM_SECONDS:
        fn(i)
        i += 1
        if i >= warmup and i % 16 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()


def time_steps(fn, steps, warmup, torch):
    """Runs warmup untimed steps (warm_up), then times exactly `steps` steps between synchronisations with
    events on the stream the kernels are launched on (torch's current stream). Returns seconds per step."""
    warm_up(fn, warmup, torch)
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(steps):
        fn(i)
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / 1e3 / steps


# ---------------------------------------------------------------- workloads

def time_steps_graph(fn, steps, warmup, torch):
    """As time_steps, but the `steps` timed steps are captured once into a HIP graph and replayed, as the
    reference replays its one-token decode step (src/cuda.rs:8686-8712): the time is the GPU's, not the
    Python launch path's. The graph is replayed untimed (upload, then warm_up's time) before the timed
    replay."""
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(steps):
            fn(i)
    warm_up(lambda i: g.replay(), 1, torch)
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    g.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / 1e3 / steps


def decode_workload(torch, gi_attn, dev, ctx, n_heads, n_kv, n_tok, steps, warmup, seed, layout="head_major",
                    i8=False, hd=HD):
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    # K+V bytes of one step: every key row once (int8 rows plus their two f32 scales)
    kv_bytes = (2 * ctx * n_kv * (hd // 2 + hd // 16) if i8 == "q4" else 2 * ctx * n_kv * (hd + 4) if i8
                else 2 * ctx * n_kv * hd * 2)
    layers = max(1, math.ceil(512e6 / kv_bytes))  # > 256 MB Infinity Cache in total
    caches = [seeded_cache(gen, ctx, n_kv, dev, torch, layout, i8, hd) for _ in range(layers)]
    q = torch.randn((n_tok, n_heads * hd), generator=gen, device=dev, dtype=torch.float32)
    out = torch.empty((n_tok, n_heads * hd), device=dev, dtype=torch.float32)
    pos0 = ctx - n_tok
    ws = gi_attn.new_workspace(ctx, n_tok, n_heads, n_kv, hd=hd, device=dev)

    def step(i):
        k, v, ks, vs = caches[i % layers]
        if i8 == "q4":
            gi_attn.decode_q4(q, k, v, ks, vs, pos0, n_heads, n_kv, out=out, workspace=ws, kv_layout=layout)
        else:
            gi_attn.decode(q, k, v, pos0, n_heads, n_kv, hd=hd, out=out, workspace=ws, kv_layout=layout, k_scale=ks,
                           v_scale=vs)

    t = time_steps_graph(step, steps, warmup, torch)
    return {"seconds": t, "bytes": kv_bytes, "layers": layers, "q": q, "cache": caches[0], "pos0": pos0,
            "layout": layout, "step": step, "ws": ws}


def prefill_flops(n, pos0, n_heads, hd=HD):
    # QK^T and PV, 2 flops per multiply-add, causal: query i sees pos0 + i + 1 keys
    keys = n * pos0 + n * (n + 1) // 2
    return 4 * n_heads * hd * keys


def prefill_workload(torch, gi_attn, dev, n, n_heads, n_kv, steps, warmup, seed, i8=False, hd=HD, f32=False):
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    q = torch.randn((n, n_heads * hd), generator=gen, device=dev, dtype=torch.float32).half()
    k, v, ks, vs = seeded_cache(gen, n, n_kv, dev, torch, i8=i8, hd=hd)
    out = torch.empty((n, n_heads * hd), device=dev, dtype=torch.float16)
    # the int8 and 4-bit caches: the keys widened into a workspace first (one launch of gi_kv_widen per step, inside
    # the timed step), then staged as the f16 cache's tiles are
    ws = gi_attn.prefill_workspace(n, n_kv, hd, 2 if i8 == "q4" else 1, dev) if i8 else None

    def step(i):
        if i8 == "q4":
            gi_attn.prefill_q4(q, k, v, ks, vs, 0, n_heads, n_kv, out=out, workspace=ws)
        else:
            gi_attn.prefill(q, k, v, 0, n_heads, n_kv, hd=hd, out=out, k_scale=ks, v_scale=vs, workspace=ws, f32=f32)

    t = time_steps(step, steps, warmup, torch)
    return {"seconds": t, "flops": prefill_flops(n, 0, n_heads, hd), "step": step, "q": q, "k": k, "v": v}


def qkrope_workload(torch, gi_attn, dev, n, n_heads, n_kv, steps, warmup, seed):
    """layer_attn's qk_norm_rope step (RMSNorm + RoPE of q and k, K/V into the f16 cache) for n tokens."""
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    row = (n_heads + 2 * n_kv) * HD
    qkv0 = torch.randn((n, row), generator=gen, device=dev, dtype=torch.float32)
    qkv = qkv0.clone()
    k = torch.empty((n, n_kv, HD), device=dev, dtype=torch.float16)
    v = torch.empty_like(k)
    qn = torch.rand(HD, generator=gen, device=dev) + 0.5
    kn = torch.rand(HD, generator=gen, device=dev) + 0.5

    def step(i):
        gi_attn.qk_norm_rope(qkv, k, v, 0, n_heads, n_kv, qn=qn, kn=kn, base=1e6)

    t = time_steps(step, steps, warmup, torch)
    # bytes the step must move: every qkv row read, the q and k heads written back, K and V rows stored (f16)
    nbytes = n * row * 4 + n * (n_heads + n_kv) * HD * 4 + 2 * n * n_kv * HD * 2
    return {"seconds": t, "bytes": nbytes, "step": step}


def chunked_workload(torch, gi_attn, dev, total, chunk, n_heads, n_kv, seed):
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    k, v, _, _ = seeded_cache(gen, total, n_kv, dev, torch)
    q = torch.randn((total, n_heads * HD), generator=gen, device=dev, dtype=torch.float32).half()
    out = torch.empty((total, n_heads * HD), device=dev, dtype=torch.float16)
    events = []
    for c0 in range(0, total, chunk):  # warm-up pass
        gi_attn.prefill(q[c0:c0 + chunk], k, v, c0, n_heads, n_kv, out=out[c0:c0 + chunk])
    torch.cuda.synchronize()
    for c0 in range(0, total, chunk):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        gi_attn.prefill(q[c0:c0 + chunk], k, v, c0, n_heads, n_kv, out=out[c0:c0 + chunk])
        e1.record()
        events.append((c0, e0, e1))
    torch.cuda.synchronize()
    per_chunk = []
    for c0, e0, e1 in events:
        s = e0.elapsed_time(e1) / 1e3
        per_chunk.append((c0, s, prefill_flops(chunk, c0, n_heads) / s / 1e12))
    return per_chunk


def hbm_copy_gbs(torch, dev):
    """Measured device copy bandwidth (read + write bytes / time) of a 1 GiB buffer: a sanity figure beside
    the published peak."""
    a = torch.empty(1 << 28, dtype=torch.float32, device=dev)
    b = torch.empty_like(a)
    t = time_steps(lambda i: b.copy_(a), 10, 3, torch)
    return 2 * a.numel() * 4 / t / 1e9


def peak_probes(torch, dev, reps=5):
    """The box's own peaks, from the probe kernels of ghost-infer_amd/gi_probes_gfx950.hsaco (built beside
    the library): the dense f16 MFMA rate (v_mfma_f32_32x32x16_f16 alone, two waves per SIMD) and an HBM
    read stream (contiguous chunks per workgroup, 16 16-byte streaming loads in flight per lane) over 1 GiB
    and over config 2's 134 MB (three buffers in turn, past the 256 MB Infinity Cache), and the LDS read rate of
    ds_read_b128 and of the transposing ds_read_b64_tr_b16 at 8 waves per CU (TB/s over all CUs). Medians over
    `reps` timings with events on torch's current stream."""
    import ctypes
    path = os.path.join(ROOT, "ghost-infer_amd", "gi_probes_gfx950.hsaco")
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is not built (run __graft_entry__.build())")
    hip = ctypes.CDLL("libamdhip64.so")
    mod = ctypes.c_void_p()
    if hip.hipModuleLoad(ctypes.byref(mod), path.encode()):
        raise RuntimeError("hipModuleLoad of the probe code object failed")
    fns = {}
    for name in ("gi_probe_mfma", "gi_probe_mfma_rand", "gi_probe_read", "gi_probe_lds"):
        f = ctypes.c_void_p()
        if hip.hipModuleGetFunction(ctypes.byref(f), mod, name.encode()):
            raise RuntimeError(f"probe kernel {name} not found")
        fns[name] = f
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def launch(f, grid, args):
        buf = ctypes.create_string_buffer(bytes(args), len(bytes(args)))
        sz = ctypes.c_size_t(len(bytes(args)))
        cfg = (ctypes.c_void_p * 5)(ctypes.c_void_p(1), ctypes.cast(buf, ctypes.c_void_p), ctypes.c_void_p(2),
                                    ctypes.cast(ctypes.pointer(sz), ctypes.c_void_p), ctypes.c_void_p(3))
        if hip.hipModuleLaunchKernel(f, grid, 1, 1, 256, 1, 1, 0, stream, None, cfg):
            raise RuntimeError("probe launch failed")

    def timed(fn, inner=1):
        # seconds per launch: `inner` launches back to back between two events, so that the host's launch
        # latency stays off short kernels
        ts = []
        for _ in range(reps + 1):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(inner):
                fn()
            e1.record()
            torch.cuda.synchronize()
            ts.append(e0.elapsed_time(e1) / 1e3 / inner)
        ts = sorted(ts[1:])
        return ts[len(ts) // 2]

    class MfmaArgs(ctypes.Structure):
        _fields_ = [("iters", ctypes.c_int), ("pad", ctypes.c_int), ("out", ctypes.c_void_p)]

    class ReadArgs(ctypes.Structure):
        _fields_ = [("p", ctypes.c_void_p), ("n16", ctypes.c_longlong), ("out", ctypes.c_void_p)]

    wgs, iters = 512, 4000  # 2048 waves: two per SIMD
    sink = torch.zeros(wgs * 256, dtype=torch.float32, device=dev)
    t = timed(lambda: launch(fns["gi_probe_mfma"], wgs, MfmaArgs(iters, 0, sink.data_ptr())))
    mfma_tflops = wgs * 4 * iters * 32 * 32768 / t / 1e12
    res = {"mfma_f16_dense_TFLOPs": round(mfma_tflops, 1)}
    # the same over operands that change every instruction, as N(0,1) data does
    t = timed(lambda: launch(fns["gi_probe_mfma_rand"], wgs, MfmaArgs(iters, 0, sink.data_ptr())))
    res["mfma_f16_dense_random_operands_TFLOPs"] = round(wgs * 4 * iters * 32 * 32768 / t / 1e12, 1)
    flag = torch.zeros(1, dtype=torch.int32, device=dev)
    for label, nbytes, rd_wgs in (("hbm_read_GBs_1GiB", 1 << 30, 1024), ("hbm_read_GBs_134MB", 134217728, 256)):
        bufs = [torch.empty(nbytes, dtype=torch.uint8, device=dev) for _ in range(3)]  # rotate past the 256 MB cache
        k = [0]

        def one():
            b = bufs[k[0] % len(bufs)]
            k[0] += 1
            launch(fns["gi_probe_read"], rd_wgs, ReadArgs(b.data_ptr(), nbytes // 16 // rd_wgs, flag.data_ptr()))
        res[label] = round(nbytes / timed(one, inner=24) / 1e9, 1)
        del bufs
    res["hbm_copy_GBs_1GiB"] = round(hbm_copy_gbs(torch, dev), 1)

    class LdsArgs(ctypes.Structure):
        _fields_ = [("iters", ctypes.c_int), ("tr", ctypes.c_int), ("out", ctypes.c_void_p)]

    # LDS operand reads at 8 waves per CU (the prefill kernels' occupancy): 512 workgroups of 4 waves
    lds_wgs, lds_iters = 512, 2000
    for label, tr, per_lane in (("lds_read_b128_TBs", 0, 16), ("lds_read_tr16_b64_TBs", 1, 8)):
        t = timed(lambda: launch(fns["gi_probe_lds"], lds_wgs, LdsArgs(lds_iters, tr, flag.data_ptr())))
        res[label] = round(lds_wgs * 256 * lds_iters * 16 * per_lane / t / 1e12, 1)
    return res


# ---------------------------------------------------------------- CPU baseline (the oracle)

def cpu_threads():
    """(all, half, logical, model): the worker counts of the CPU baseline. "all" is the CPUs this process may
    run on (its affinity mask), capped at 16, the host share of one GPU on the benchmark boxes; "half" is
    logical/2 of that, the reference's default thread count (src/main.rs:122-125)."""
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = os.cpu_count() or 1
    n = max(1, min(16, avail))
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return n, max(1, n // 2), os.cpu_count() or avail, model


def _median_time(fn, budget_s, min_runs=5, max_runs=200):
    fn()  # warm-up
    times = []
    t_end = time.time() + budget_s
    while time.time() < t_end or len(times) < min_runs:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
        if len(times) >= max_runs:
            break
    times.sort()
    return times[len(times) // 2], len(times)


def _ref_layout_f32(k, v, n_kv):
    """K/V caches (torch, f16, reference or head-major layout) as f32 numpy rows [pos, n_kv*hd]: the
    reference's CPU session holds an f32 cache (src/model.rs:1326-1327); the widening is exact."""
    if k.dim() == 3 and k.shape[0] == n_kv and k.shape[1] != n_kv:  # head-major: to [pos][n_kv][hd]
        k, v = k.transpose(0, 1), v.transpose(0, 1)
    kn = k.float().contiguous().cpu().numpy()
    vn = v.float().contiguous().cpu().numpy()
    return kn.reshape(kn.shape[0], -1), vn.reshape(vn.shape[0], -1)


def cpu_baseline_decode(q, cache, pos0, n_heads, n_kv, threads, budget_s=8.0):
    """The oracle's restatement of Model::attention (src/model.rs:1320-1409) for the same decode (q, cache) on
    an f32 cache, with `threads` workers: (median seconds, runs)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import gi_oracle

    qn = q.cpu().numpy()
    kn, vn = _ref_layout_f32(cache[0], cache[1], n_kv)
    return _median_time(lambda: gi_oracle.attention(qn, kn, vn, pos0, n_heads, n_kv, threads=threads), budget_s)


def cpu_baseline_prefill(q, k, v, n_heads, n_kv, threads, rows=64, budget_s=8.0):
    """The oracle's Model::attention on a bounded sample of the causal prefill: the last `rows` query rows of
    the prompt (each sees nearly the whole prompt), all heads, over the same cache widened to f32. Returns
    (TFLOP/s, runs, sample flops, median seconds)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import gi_oracle

    n = q.shape[0]
    pos0 = n - rows
    qn = q[pos0:].float().cpu().numpy()
    kn, vn = _ref_layout_f32(k, v, n_kv)
    t, runs = _median_time(lambda: gi_oracle.attention(qn, kn, vn, pos0, n_heads, n_kv, threads=threads), budget_s,
                           min_runs=3, max_runs=50)
    flops = prefill_flops(rows, pos0, n_heads)
    return flops / t / 1e12, runs, flops, t


def prefill_roofline(gi_attn, r, steps, torch, profile="pmc_prefill_prefill8k", kernel="gi_prefill_fwd",
                     peak=None):
    """Roofline object of the prefill kernel: algorithmic flops of one launch / its mean duration, against the
    dense f16 MFMA peak (the f32 kernels: the dense f32 MFMA peak)."""
    peak = peak or F16_DENSE_PEAK_TFLOPS
    # ~0.1 s of launches before the timed ones (at most 100)
    warm = min(100, max(0, math.ceil(0.1 / r["seconds"])))
    kt = kernel_times(gi_attn, r["step"], steps, torch, ("prefill", "kv_widen"), warm)
    ms, n = kt["prefill"]
    tf = r["flops"] / (ms / 1e3) / 1e12
    line = {"bound": "mfma", "achieved": round(tf, 1), "peak": peak, "unit": "TFLOP/s",
            "frac": round(tf / peak, 4), "traffic": profile_traffic(profile),
            "kernel": kernel, "algorithmic_flops_per_launch": r["flops"],
            "kernel_ms_per_launch": round(ms, 5), "launches_timed": n}
    if kt["kv_widen"][1]:  # the int8 / 4-bit cache's widening launch, part of every step
        line["widen_ms_per_launch"] = round(kt["kv_widen"][0], 5)
    return line


# ---------------------------------------------------------------- one line per workload

DECODE_WORKLOADS = {
    # name: (ctx, n_heads, n_kv, n_tok, hd, int8, description)
    "decode64k": (65536, 32, 4, 1, 128, False, "config 2: decode, 1 token, ctx 65536, 32q/4kv, hd 128"),
    "decode4k": (4096, 32, 8, 1, 128, False, "config 1: decode, 1 token, ctx 4096, 32q/8kv, hd 128"),
    "decode4k_i8": (4096, 32, 8, 1, 128, True, "config 1 over the int8 cache: decode, 1 token, ctx 4096, 32q/8kv"),
    "decode4k_h64": (4096, 32, 8, 1, 64, False, "config 1's shape with 64-wide heads: decode, 1 token, ctx 4096, 32q/8kv"),
    "decode4k_h256": (4096, 16, 2, 1, 256, False, "decode with 256-wide heads (16q/2kv), 1 token, ctx 4096, f16 cache"),
    "decode4k_h256_i8": (4096, 16, 2, 1, 256, True, "decode with 256-wide heads (16q/2kv), 1 token, ctx 4096, int8 cache"),
    "verify": (32776, 32, 4, 8, 128, False, "config 4: verify, 8 tokens at a 32768-key prefix, 32q/4kv, hd 128"),
    "decode64k_i8": (65536, 32, 4, 1, 128, True, "config 2 over the int8 cache: decode, 1 token, ctx 65536, 32q/4kv"),
    "verify_i8": (32776, 32, 4, 8, 128, True, "config 4 over the int8 cache: verify, 8 tokens at 32768, 32q/4kv"),
    "decode64k_h256": (65536, 16, 2, 1, 256, False, "decode with 256-wide heads (Qwen3.5-style 16q/2kv), 1 token, "
                                                    "ctx 65536, f16 cache"),
    "verify_h256": (32776, 16, 2, 8, 256, False, "verify with 256-wide heads (Qwen3.5-style 16q/2kv), 8 tokens at a "
                                                 "32768-key prefix, f16 cache"),
    "decode64k_h256_i8": (65536, 16, 2, 1, 256, True, "decode with 256-wide heads over the int8 cache (Qwen3.5/3.6-style "
                                                      "16q/2kv, the reference's attention_decode_tc256), 1 token, ctx 65536"),
    "verify_h256_i8": (32776, 16, 2, 8, 256, True, "verify with 256-wide heads over the int8 cache, 8 tokens at a "
                                                   "32768-key prefix, 16q/2kv"),
    "decode64k_h256_q4": (65536, 16, 2, 1, 256, "q4", "decode with 256-wide heads over the 4-bit cache (the "
                                                      "reference's --kv q4), 1 token, ctx 65536, 16q/2kv"),
    "verify_h256_q4": (32776, 16, 2, 8, 256, "q4", "verify with 256-wide heads over the 4-bit cache, 8 tokens at a "
                                                   "32768-key prefix, 16q/2kv"),
    "decode64k_h64": (65536, 32, 8, 1, 64, False, "decode with 64-wide heads (Llama-3.2-1B-style 32q/8kv), 1 token, "
                                                  "ctx 65536, f16 cache"),
    "decode64k_h64_i8": (65536, 32, 8, 1, 64, True, "decode with 64-wide heads over the int8 cache, 1 token, ctx "
                                                    "65536, 32q/8kv"),
    "decode16k_h80": (16384, 32, 32, 1, 80, False, "decode with 80-wide heads (Phi-2-style 32q/32kv, the f32 kernels), "
                                                   "1 token, ctx 16384, f16 cache"),
    "decode16k_h80_i8": (16384, 32, 32, 1, 80, True, "decode with 80-wide heads over the int8 cache (the f32 kernels), "
                                                     "1 token, ctx 16384, 32q/32kv"),
}


def run_decode(torch, gi_attn, dev, w, steps, warmup, n_tok_override=None, reference_layout=False):
    """One decode workload: the line's fields, plus the workload's tensors for a CPU baseline."""
    ctx, n_heads, n_kv, n_tok, hd, i8, cfg = DECODE_WORKLOADS[w]
    if n_tok_override and w.startswith("verify") and n_tok_override != n_tok:
        ctx, n_tok = 32768 + n_tok_override, n_tok_override
        cfg = f"config 4's shape with {n_tok} tokens per block" + (" over the int8 cache" if i8 else "")
    log(f"[bench] {cfg}")
    r = decode_workload(torch, gi_attn, dev, ctx, n_heads, n_kv, n_tok, steps, warmup, 1234, i8=i8, hd=hd)
    gbs = r["bytes"] / r["seconds"] / 1e9
    chunk, nsplit = gi_attn.decode_plan(ctx, n_tok, n_heads, n_kv, hd)
    if i8:  # the plan query is the f16 cache's; the int8 and 4-bit kernels' pair groups (and tiles) differ
        chunk = nsplit = None
        if (hd == 128 and i8 is True and n_tok * n_heads // n_kv <= 8) or (hd == 256 and n_tok * n_heads // n_kv <= 16):
            # the plan of these kernels' single pair group: slices of whole wave tiles (64 int8 keys at head size 128,
            # 16 keys at 256), at least one tile per wave
            tile = 64 if hd == 128 else 16
            least = -(-ctx // max(1, 256 // n_kv))
            chunk = max(4 * tile, -(-least // tile) * tile)
    kt = kernel_times(gi_attn, r["step"], steps, torch, ("decode_partial", "decode_combine"))
    part_ms, part_n = kt["decode_partial"]
    comb_ms, _ = kt["decode_combine"]
    # algorithmic bytes of one split-kernel launch: K and V of every span key and the queries (the slice
    # partials it writes are overhead of the split, not counted)
    part_bytes = r["bytes"] + n_tok * n_heads * hd * 4
    kern_gbs = part_bytes / (part_ms / 1e3) / 1e9
    line = {
        "value": round(gbs, 1), "unit": "GB/s", "ms_per_step": r["seconds"] * 1e3,
        "dtype": ("4-bit K/V + f16 scales, f32 math" if i8 == "q4" else "int8 K/V + f32 scales, f32 math" if i8
                  else "f16 K/V, f32 math"),
        "config": {"workload": cfg, "ctx": ctx, "n_tok": n_tok, "n_heads": n_heads, "n_kv": n_kv, "hd": hd,
                   "kv_bytes_per_step": r["bytes"], "layers_rotated": r["layers"],
                   "slices": nsplit, "keys_per_slice": chunk, "kv_layout": f"head_major [n_kv][ctx][{hd}]"},
        "roofline": {"bound": "hbm", "achieved": round(kern_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(kern_gbs / HBM_PEAK_GBS, 4), "traffic": profile_traffic(f"pmc_decode_partial_{w}"),
                     "kernel": decode_kernel_name(n_tok, n_heads, n_kv, hd, i8, chunk) + " (split-K pass)",
                     "algorithmic_bytes_per_launch": part_bytes,
                     "kernel_ms_per_launch": round(part_ms, 5), "launches_timed": part_n,
                     "combine_ms_per_launch": round(comb_ms, 5) if comb_ms else None,
                     "step_frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)},
    }
    if reference_layout and not i8 and hd == HD:
        # the same decode over caches in the reference's [position][n_kv][128] layout
        r_ref = decode_workload(torch, gi_attn, dev, ctx, n_heads, n_kv, n_tok, steps, warmup, 1234,
                                layout="reference")
        line["config"]["reference_layout_GBs"] = round(r_ref["bytes"] / r_ref["seconds"] / 1e9, 1)
        line["config"]["reference_layout_ms_per_step"] = r_ref["seconds"] * 1e3
        del r_ref
    return line, r


PREFILL_WORKLOADS = ("prefill8k", "prefill8k_i8", "prefill8k_h256", "prefill8k_h256_i8", "prefill8k_h256_q4",
                     "prefill8k_h64", "prefill8k_h64_i8", "prefill8k_h96", "prefill8k_h96_i8", "prefill8k_f32")


def run_prefill(torch, gi_attn, dev, w, steps, warmup):
    i8 = "q4" if w.endswith("_q4") else w.endswith("_i8")
    hd = 256 if "_h256" in w else 64 if "_h64" in w else 96 if "_h96" in w else HD
    nh, nkv = (16, 2) if hd == 256 else (32, 32) if hd == 96 else (32, 8)
    cache = " over the 4-bit cache" if i8 == "q4" else " over the int8 cache" if i8 else ""
    log(f"[bench] causal prefill 8192 tokens, {nh}q/{nkv}kv, hd {hd}{cache}")
    f32 = w == "prefill8k_f32"  # config 3's prompt in f32 (the reference's GHOST_INFER_NO_TC_ATT)
    r = prefill_workload(torch, gi_attn, dev, 8192, nh, nkv, steps, warmup, 99, i8=i8, hd=hd, f32=f32)
    tf = r["flops"] / r["seconds"] / 1e12
    # (the int8 cache: the kernels staging the pre-widened keys, *_i8s; the 4-bit cache widened runs the f16 kernel)
    kernel = ("gi_prefill_fwd_h256r" + ("_i8s" if i8 is True else "") if hd == 256
              else "gi_prefill_fwd_h64" + ("_i8s" if i8 else "") if hd == 64
              else "gi_prefill_f32" + ("_i8" if i8 else "") + f"_h{hd}" if hd not in (64, 128)
              else "gi_prefill_f32_h128" if f32
              else "gi_prefill_fwd_i8s" if i8 else "gi_prefill_fwd")
    line = {
        "value": round(tf, 1), "unit": "TFLOP/s", "ms_per_step": r["seconds"] * 1e3,
        "dtype": ("4-bit K/V widened to f16 MFMA, f32 acc" if i8 == "q4" else
                  "f32 MFMA (" + ("int8" if i8 else "f16") + " cache widened), f32 acc" if hd not in (64, 128, 256) or f32
                  else
                  "int8 K/V widened to f16 MFMA, f32 acc" if i8 else "f16 MFMA, f32 acc"),
        "config": {"workload": (f"causal prefill, 8192 tokens, {nh}q/{nkv}kv, hd 256 (Qwen3.5-style heads){cache}"
                                if hd == 256 else
                                f"causal prefill, 8192 tokens, 32q/8kv, hd 64 (Llama-3.2-1B-style heads){cache}"
                                if hd == 64 else
                                "causal prefill, 8192 tokens, 32q/32kv, hd 96 (Phi-3-style heads, the f32 kernels)" + cache
                                if hd == 96 else "config 3's prompt in f32 (no f16 Q or P: GHOST_INFER_NO_TC_ATT)"
                                if f32 else "config 3: causal prefill, 8192 tokens, 32q/8kv, hd 128" +
                                (", int8 cache" if i8 else "")), "flops_per_step": r["flops"]},
        "roofline": prefill_roofline(gi_attn, r, steps, torch, f"pmc_prefill_{w}", kernel,
                                     FP32_DENSE_PEAK_TFLOPS if hd not in (64, 128, 256) or f32 else None),
    }
    return line, r


def run_chunked(torch, gi_attn, dev):
    log("[bench] config 5: chunked prefill 131072 in 2048 chunks, 32q/4kv")
    per = chunked_workload(torch, gi_attn, dev, 131072, 2048, 32, 4, 5)
    total = sum(s for _, s, _ in per)
    flops = sum(prefill_flops(2048, c0, 32) for c0, _, _ in per)
    tf = flops / total / 1e12
    return {
        "value": round(tf, 1), "unit": "TFLOP/s", "ms_per_step": total * 1e3, "steps": len(per),
        "dtype": "f16 MFMA, f32 acc",
        "config": {"workload": "config 5: chunked prefill, 131072 tokens in 2048 chunks, 32q/4kv",
                   "total_seconds": total, "total_flops": flops,
                   "per_chunk_tflops": [round(t, 1) for _, _, t in per]},
        # one launch per chunk, timed by events around it: the roofline is the whole prefill's flops over the
        # sum of its launches (the chunks' own figures are in per_chunk_tflops)
        "roofline": {"bound": "mfma", "achieved": round(tf, 1), "peak": F16_DENSE_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tf / F16_DENSE_PEAK_TFLOPS, 4), "traffic": profile_traffic("pmc_prefill_chunked"),
                     "kernel": "gi_prefill_fwd", "algorithmic_flops_per_launch": flops // len(per),
                     "kernel_ms_per_launch": round(total * 1e3 / len(per), 5), "launches_timed": len(per)},
    }


def run_qkrope(torch, gi_attn, dev, steps, warmup):
    log("[bench] qk_norm_rope + KV store for 8192 tokens, 32q/8kv (the cache write of config 3)")
    r = qkrope_workload(torch, gi_attn, dev, 8192, 32, 8, steps, warmup, 7)
    gbs = r["bytes"] / r["seconds"] / 1e9
    ms, n_l = kernel_times(gi_attn, r["step"], steps, torch, ("qk_norm_rope",))["qk_norm_rope"]
    kern = r["bytes"] / (ms / 1e3) / 1e9
    return {
        "value": round(gbs, 1), "unit": "GB/s", "ms_per_step": r["seconds"] * 1e3, "dtype": "f32 math, f16 cache",
        "config": {"workload": "qk_norm_rope + f16 KV store, 8192 tokens, 32q/8kv, hd 128", "bytes_per_step": r["bytes"]},
        "roofline": {"bound": "hbm", "achieved": round(kern, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(kern / HBM_PEAK_GBS, 4), "traffic": profile_traffic("pmc_qk_norm_rope_qkrope"),
                     "kernel": "gi_qk_norm_rope",
                     "algorithmic_bytes_per_launch": r["bytes"], "kernel_ms_per_launch": round(ms, 5),
                     "launches_timed": n_l},
    }


ROOF_KEEP = ("bound", "achieved", "peak", "unit", "frac", "traffic")


def compact_roofline(rf, extra=()):
    return {k: rf[k] for k in ROOF_KEEP + tuple(extra) if k in rf}


def compact_line(result):
    """The printed line: the headline fields, its roofline and CPU baseline, and for each other benchmark config
    (1, 3, 4 and 5) its value, time and roofline; every other workload's roofline fraction. The full record
    (every field, every workload) goes to the detail file. Kept near 2 KB so that a record holding only the
    end of the output still holds all of it."""
    out = {k: result[k] for k in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step",
                                  "higher_is_better", "scaling", "vs_baseline", "dtype", "data") if k in result}
    if isinstance(out.get("ms_per_step"), float):
        out["ms_per_step"] = round(out["ms_per_step"], 6)
    cfg = result.get("config", {})
    out["config"] = {k: cfg[k] for k in ("workload", "ctx", "n_tok", "n_heads", "n_kv", "hd", "slices") if k in cfg}
    if "roofline" in result:
        out["roofline"] = compact_roofline(result["roofline"], ("kernel_ms_per_launch",
                                                                "combine_ms_per_launch", "step_frac_of_hbm_peak"))
    cb = result.get("cpu_baseline")
    if cb:
        out["cpu_baseline"] = {k: cb[k] for k in ("value", "unit", "cores", "kind") if k in cb}
        out["cpu_baseline"]["sample"] = cb.get("sample_short", cb.get("sample", ""))[:120]
    sec = result.get("secondary")
    if sec:
        cs = {}
        for w in ("decode4k", "verify", "prefill8k", "chunked"):
            if w in sec:
                e = sec[w]
                cs[w] = {"value": e["value"], "unit": e["unit"], "ms_per_step": round(e["ms_per_step"], 5),
                         "roofline": compact_roofline(e["roofline"])}
                if w == "chunked":
                    c = e["config"]
                    cs[w]["total_s"] = round(c["total_seconds"], 5)
                    pc = c["per_chunk_tflops"]
                    # every 16th chunk (chunk index 16i) and the last; all of them are in the detail file
                    cs[w]["per_chunk_tflops_every16"] = [round(t) for t in pc[::16]] + [round(pc[-1])]
        pk = sec.get("peaks_measured")
        if isinstance(pk, dict):
            # this box's measured ceilings: MFMA over constant and over changing operands, the 134 MB read
            cs["peaks"] = {short: pk[k] for short, k in (("mfma_TF", "mfma_f16_dense_TFLOPs"),
                                                         ("mfma_rand_TF", "mfma_f16_dense_random_operands_TFLOPs"),
                                                         ("read134_GBs", "hbm_read_GBs_134MB")) if k in pk}
        # "workload=frac ..." in one string: the shortest form that keeps every name
        cs["frac_other"] = " ".join(f"{w}={sec[w]['roofline']['frac']:.3f}" for w in sec
                                    if w not in cs and isinstance(sec[w], dict) and "roofline" in sec[w])
        out["secondary"] = cs
    return out


def secondary_entry(line):
    """The fields of a workload's line that a secondary entry keeps."""
    keep = ("value", "unit", "ms_per_step", "dtype", "config", "roofline", "steps")
    return {k: line[k] for k in keep if k in line}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="decode64k",
                    choices=[*DECODE_WORKLOADS, *PREFILL_WORKLOADS, "chunked", "qkrope", "peaks"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--n-tok", type=int, default=None,
                    help="verify workloads: draft tokens per block (default 8, config 4's)")
    ap.add_argument("--reference-layout", action="store_true",
                    help="decode workloads: also time the reference's cache layout")
    ap.add_argument("--verbose", action="store_true", help="progress messages on stderr")
    ap.add_argument("--detail-out", default="",
                    help="file for the full record (every field of every workload); none by default")
    ap.add_argument("--full-line", action="store_true", help="print the full record instead of the compact line")
    args = ap.parse_args()
    global VERBOSE
    VERBOSE = VERBOSE or args.verbose
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path (asked for {args.gpus})",
              file=sys.stderr)
        sys.exit(2)

    import torch

    import gi_attn

    dev = torch.device("cuda:0")
    quiet_fd2 = None
    if not VERBOSE:
        # the device's first initialisation prints a libdrm notice on stderr; keep it out of the output's tail
        sys.stderr.flush()
        quiet_fd2 = os.dup(2)
        devnull = os.open(os.devnull, os.O_WRONLY)
        os.dup2(devnull, 2)
        os.close(devnull)
    try:
        torch.zeros(1, device=dev)
        gi_attn.init()
    finally:
        if quiet_fd2 is not None:
            os.dup2(quiet_fd2, 2)
            os.close(quiet_fd2)
    result = {"metric": METRIC, "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
              "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "data": "synthetic"}
    w = args.workload
    cpu = None  # (kind of workload, workload tensors) for the CPU baseline
    if w == "peaks":
        log("[bench] peak probes: dense f16 MFMA rate, HBM read stream, device copy")
        pk = peak_probes(torch, dev)
        result.update({"value": pk["mfma_f16_dense_TFLOPs"], "unit": "TFLOP/s", "ms_per_step": None,
                       "dtype": "f16 MFMA, f32 acc", "config": {"workload": "peak probes of this box", **pk},
                       "roofline": {"bound": "mfma", "achieved": pk["mfma_f16_dense_TFLOPs"],
                                    "peak": F16_DENSE_PEAK_TFLOPS, "unit": "TFLOP/s",
                                    "frac": round(pk["mfma_f16_dense_TFLOPs"] / F16_DENSE_PEAK_TFLOPS, 4),
                                    "traffic": None, "kernel": "gi_probe_mfma"}})
    elif w in DECODE_WORKLOADS:
        line, r = run_decode(torch, gi_attn, dev, w, args.steps, args.warmup, args.n_tok, args.reference_layout)
        result.update(line)
        if not DECODE_WORKLOADS[w][5] and DECODE_WORKLOADS[w][4] == HD:
            cpu = ("decode", w, r)
    elif w == "qkrope":
        result.update(run_qkrope(torch, gi_attn, dev, args.steps, args.warmup))
    elif w in PREFILL_WORKLOADS:
        line, r = run_prefill(torch, gi_attn, dev, w, args.steps, args.warmup)
        result.update(line)
        if w == "prefill8k":
            cpu = ("prefill", w, r)
    else:
        result.update(run_chunked(torch, gi_attn, dev))

    sec_r = {}
    if w == "decode64k" and not args.no_secondary:
        # every other config of the benchmark on the same line, each with its own roofline
        sec = {}
        steps2, warm2 = max(20, args.steps // 4), max(5, args.warmup // 2)
        for w2 in ("decode4k", "verify"):
            line, r2 = run_decode(torch, gi_attn, dev, w2, steps2, warm2)
            sec[w2] = secondary_entry(line)
            if w2 == "decode4k":
                sec_r["decode4k"] = r2
            del r2
        line, r2 = run_prefill(torch, gi_attn, dev, "prefill8k", 30, 10)
        sec["prefill8k"] = secondary_entry(line)
        sec_r["prefill8k"] = r2
        sec["chunked"] = secondary_entry(run_chunked(torch, gi_attn, dev))
        # the cache formats and head sizes beyond the configs: int8, head size 256 over f16, int8 and 4 bits
        for w2 in ("decode64k_i8", "verify_i8", "decode64k_h256", "verify_h256", "decode64k_h256_i8",
                   "verify_h256_i8", "decode64k_h256_q4", "verify_h256_q4", "decode64k_h64", "decode64k_h64_i8"):
            line, r2 = run_decode(torch, gi_attn, dev, w2, steps2, warm2)
            sec[w2] = secondary_entry(line)
            del r2
        for w2 in ("prefill8k_i8", "prefill8k_h256", "prefill8k_h256_i8", "prefill8k_h256_q4", "prefill8k_h64",
                   "prefill8k_h64_i8"):
            line, r2 = run_prefill(torch, gi_attn, dev, w2, 20, 5)
            sec[w2] = secondary_entry(line)
            del r2
        sec["hbm_copy_measured_GBs"] = round(hbm_copy_gbs(torch, dev), 1)
        sec["peaks_measured"] = peak_probes(torch, dev)
        result["secondary"] = sec

    if cpu and not args.no_cpu_baseline:
        # the reference's CPU attention (the oracle's restatement of Model::attention, f32 cache) on this
        # host, at all of its CPU share and at logical/2 (the reference's default thread count)
        n_all, n_half, logical, model = cpu_threads()
        kind, cw, r = cpu
        ctx, nh, nkv = (DECODE_WORKLOADS[cw][:3] if kind == "decode" else (8192, 32, 8))
        log(f"[bench] cpu baseline (oracle, Model::attention restatement, f32 cache) on {n_all} and {n_half} threads")
        runs = []

        def decode_runs(label, rr, nh_, nkv_):
            for th in (n_all, n_half):
                t_cpu, reps = cpu_baseline_decode(rr["q"], rr["cache"], rr["pos0"], nh_, nkv_, th)
                runs.append({"config": label, "threads": th, "value": round(rr["bytes"] / t_cpu / 1e9, 3),
                             "unit": "GB/s (K+V bytes of the f16 cache)",
                             "sample": f"{reps} runs of the whole decode (median {t_cpu * 1e3:.2f} ms/run)"})

        def prefill_runs(rr):
            for th in (n_all, n_half):
                tf_cpu, reps, fl, t_cpu = cpu_baseline_prefill(rr["q"], rr["k"], rr["v"], 32, 8, th)
                runs.append({"config": "prefill8k", "threads": th, "value": round(tf_cpu, 4), "unit": "TFLOP/s",
                             "sample": f"the last 64 of the 8192 query rows, all heads ({fl / 1e9:.1f} GFLOP), "
                                       f"{reps} runs (median {t_cpu * 1e3:.1f} ms/run)"})

        if kind == "decode":
            decode_runs(cw, r, nh, nkv)
        else:
            prefill_runs(r)
        if "decode4k" in sec_r:  # config 1 is the reference's own CPU config
            decode_runs("decode4k", sec_r["decode4k"], 32, 8)
        if "prefill8k" in sec_r:
            prefill_runs(sec_r["prefill8k"])
        head_run = runs[0]
        result["cpu_baseline"] = {
            "value": head_run["value"], "unit": head_run["unit"].split(" ")[0], "cores": head_run["threads"],
            "kind": "port",
            "sample": f"{head_run['config']}: {head_run['sample']}; the oracle's C++ restatement of Model::attention "
                      f"(src/model.rs:1320-1409) over the same inputs with the cache widened to f32",
            "sample_short": (f"{head_run['config']}: {head_run['sample'].split(' of the')[0].split(' (')[0]}, "
                             f"oracle Model::attention, f32 cache"),
            "cpu_model": model, "logical_cpus": logical,
            "threads_note": f"all = this process's CPUs capped at 16 (the host share of one GPU), half = the "
                            f"reference's default logical/2",
            "runs": runs}
    if args.detail_out:
        try:
            os.makedirs(os.path.dirname(os.path.abspath(args.detail_out)), exist_ok=True)
            with open(args.detail_out, "w") as f:
                json.dump(result, f, indent=1)
        except OSError as e:
            log(f"[bench] detail file not written: {e}")
    print(json.dumps(result) if args.full_line else json.dumps(compact_line(result), separators=(",", ":")),
          flush=True)


if __name__ == "__main__":
    main()
