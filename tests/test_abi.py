"""The C-ABI library: it loads, exports every symbol include/gi_attn.h declares, and rejects bad
arguments with a message before touching the GPU (no compute calls here)."""
import ctypes
import os
import re
import subprocess

import pytest

import gi_attn


def _fake_pointers_only_without_a_gpu():
    # These calls pass made-up device addresses and expect the host checks to refuse them before any launch.
    # With a GPU present a check that let one through would launch over those addresses, so they run only on a
    # host without one (the CPU suite).
    import torch

    if torch.cuda.is_available():
        pytest.skip("passes made-up device pointers: runs only without a GPU")

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "gi_attn.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(gi_\w+)\s*\(", text)))


def test_header_declares_the_python_symbols():
    assert declared_symbols() == sorted(gi_attn.SYMBOLS)


def test_library_exports_every_declared_symbol():
    lib = gi_attn.load_library()
    for name in declared_symbols():
        assert hasattr(lib, name), name


def test_code_object_built():
    assert os.path.getsize(gi_attn.HSACO_PATH) > 0
    # the bench's peak probes: their own code object beside it
    assert os.path.getsize(os.path.join(os.path.dirname(gi_attn.HSACO_PATH), "gi_probes_gfx950.hsaco")) > 0


def test_unsupported_head_size_is_rejected_with_message():
    lib = gi_attn.load_library()
    c, n = ctypes.c_int(), ctypes.c_int()
    rc = lib.gi_attn_decode_plan(100, 1, 32, 8, 72, ctypes.byref(c), ctypes.byref(n))
    assert rc == -1
    assert "head size 72" in lib.gi_last_error().decode()
    for hd in (64, 128, 256, 16, 32, 48, 80, 96, 112):
        assert lib.gi_attn_decode_plan(100, 1, 32, 8, hd, ctypes.byref(c), ctypes.byref(n)) == 0
    rc = lib.gi_attn_decode_plan(100, 1, 30, 8, 128, ctypes.byref(c), ctypes.byref(n))
    assert rc == -1 and "multiple of n_kv" in lib.gi_last_error().decode()


def test_decode_rejects_bad_arguments_before_any_launch():
    _fake_pointers_only_without_a_gpu()
    lib = gi_attn.load_library()
    # null tensors, hd 72, misaligned pointers: all refused on the host
    rc = lib.gi_attn_decode(None, None, 4096, None, None, 512, 128, None, 4096, None, 0, 0, None, 0, 1, 32, 4, 128,
                            0.088)
    assert rc == -1 and "null" in lib.gi_last_error().decode()
    rc = lib.gi_attn_decode(None, 16, 4096, 16, 16, 512, 128, 16, 4096, None, 0, 0, None, 0, 1, 32, 4, 72, 0.1)
    assert rc == -1 and "head size" in lib.gi_last_error().decode()
    rc = lib.gi_attn_decode(None, 8, 4096, 16, 16, 512, 128, 16, 4096, None, 0, 0, None, 0, 1, 32, 4, 128, 0.1)
    assert rc == -1 and "aligned" in lib.gi_last_error().decode()
    rc = lib.gi_attn_prefill(None, 16, 7, 4096, 16, 16, 1024, 128, 16, 0, 4096, 0, 16, 32, 8, 128, 0.1)
    assert rc == -1 and "dtypes" in lib.gi_last_error().decode()


def test_int8_entry_points_reject_bad_arguments_before_any_launch():
    _fake_pointers_only_without_a_gpu()
    lib = gi_attn.load_library()
    # int8 rows need 16-element strides, non-null 4-byte aligned scales and positive scale strides
    rc = lib.gi_attn_decode_i8(None, 16, 4096, 16, 16, 16, 16, 520, 8, 0, 0, 16, 4096, None, 0, 0, None, 0, 1, 32, 4,
                               128, 0.1)
    assert rc == -1 and "multiples of 16" in lib.gi_last_error().decode()
    rc = lib.gi_attn_decode_i8(None, 16, 4096, 16, 16, None, 16, 512, 128, 0, 0, 16, 4096, None, 0, 0, None, 0, 1, 32,
                               4, 128, 0.1)
    assert rc == -1 and "scale" in lib.gi_last_error().decode()
    rc = lib.gi_attn_decode_i8(None, 16, 4096, 16, 16, 18, 16, 512, 128, 0, 0, 16, 4096, None, 0, 0, None, 0, 1, 32,
                               4, 128, 0.1)
    assert rc == -1 and "4-byte aligned" in lib.gi_last_error().decode()
    rc = lib.gi_attn_decode_i8(None, 16, 4096, 16, 16, 16, 16, 512, 128, -4, 1, 16, 4096, None, 0, 0, None, 0, 1, 32,
                               4, 128, 0.1)
    assert rc == -1 and "sc_stride" in lib.gi_last_error().decode()
    rc = lib.gi_qk_norm_rope_i8(None, 16, None, None, 16, 16, None, None, 512, 128, 0, 0, 0, None, 0, 1, 32, 4, 128,
                                128, 1e4, None, 1, 1e-6)
    assert rc == -1 and "scale" in lib.gi_last_error().decode()


def test_device_position_needs_a_capacity():
    _fake_pointers_only_without_a_gpu()
    lib = gi_attn.load_library()
    # the cache write with a device position must be told the capacity (its kernel skips rows past it)
    rc = lib.gi_qk_norm_rope(None, 16, None, None, 16, 16, 512, 128, 0, 16, 0, 1, 32, 4, 128, 128, 1e4, None, 1, 1e-6)
    assert rc == -1 and "ctx_cap" in lib.gi_last_error().decode()
    rc = lib.gi_qk_norm_rope(None, 16, None, None, 16, 16, 512, 128, 100, None, 50, 1, 32, 4, 128, 128, 1e4, None, 1,
                             1e-6)
    assert rc == -1 and "exceed ctx_cap" in lib.gi_last_error().decode()


def test_relayout_rejects_bad_arguments_before_any_launch():
    _fake_pointers_only_without_a_gpu()
    lib = gi_attn.load_library()
    assert lib.gi_kv_relayout(None, 16, 256, 4096, 1 << 20, 256, 8192, 0, 4, 256) == 0  # nothing to copy
    rc = lib.gi_kv_relayout(None, 16, 256, 4096, 1 << 20, 256, 8192, 16, 4, 254)
    assert rc == -1 and "multiple of 4" in lib.gi_last_error().decode()
    rc = lib.gi_kv_relayout(None, 16, 256, 4096, 1 << 20, 256, -8192, 16, 4, 256)
    assert rc == -1 and "positive" in lib.gi_last_error().decode()
    # [4 heads][16 rows][256 B] at 16 into [4][32][256 B] at 4096: the spans overlap
    rc = lib.gi_kv_relayout(None, 16, 256, 4096, 4096, 256, 8192, 16, 4, 256)
    assert rc == -1 and "overlap" in lib.gi_last_error().decode()


@pytest.mark.parametrize("ctx,n_tok,n_heads,n_kv,hd", [(4096, 1, 32, 8, 128), (65536, 1, 32, 4, 128),
                                                       (32776, 8, 32, 4, 128), (100, 15, 8, 1, 128),
                                                       (1, 1, 32, 4, 128), (65536, 1, 16, 2, 256),
                                                       (32776, 8, 16, 2, 256), (5000, 15, 16, 2, 256),
                                                       (4096, 1, 9, 3, 64), (32776, 15, 9, 3, 64)])
def test_decode_plan_covers_the_span(ctx, n_tok, n_heads, n_kv, hd):
    part = (hd + 4) * 4  # bytes of one slice partial

    chunk, nsplit = gi_attn.decode_plan(ctx, n_tok, n_heads, n_kv, hd)
    # whole wave tiles (16 keys at head size 256, 32 at 128), at least one per wave of the workgroup
    assert chunk % (16 if hd == 256 else 32) == 0 and chunk >= (64 if hd == 256 else 128)
    assert (nsplit - 1) * chunk < ctx <= nsplit * chunk
    if nsplit > 1:
        # every launch of up to n_tok tokens with spans up to ctx fits the workspace size query
        need = n_tok * n_heads * nsplit * part
        assert gi_attn.workspace_bytes(ctx, n_tok, n_heads, n_kv, hd) >= need
    for span in (1, ctx // 3 + 1, ctx):
        for t in range(1, n_tok + 1):
            c2, s2 = gi_attn.decode_plan(span, t, n_heads, n_kv, hd)
            if s2 > 1:
                assert gi_attn.workspace_bytes(ctx, n_tok, n_heads, n_kv, hd) >= t * n_heads * s2 * part


def test_python_mirror_raises_without_gpu_tensors():
    import torch

    with pytest.raises(gi_attn.GiAttnError):
        gi_attn.decode(torch.zeros(1, 4096), torch.zeros(8, 512, dtype=torch.float16),
                       torch.zeros(8, 512, dtype=torch.float16), 7, 32, 4)


def test_kernel_timing_reads_and_rejects_unknown_kinds():
    lib = gi_attn.load_library()
    ms, n = ctypes.c_double(-1), ctypes.c_int(-1)
    rc = lib.gi_kernel_timing_read(b"gemm", ctypes.byref(ms), ctypes.byref(n))
    assert rc == -1 and "unknown kernel" in lib.gi_last_error().decode()
    assert lib.gi_kernel_timing_read(None, ctypes.byref(ms), ctypes.byref(n)) == -1
    # nothing launched: every kind reads as zero launches, without touching a GPU
    assert lib.gi_kernel_timing(1) == 0
    for kind in (b"decode_partial", b"decode_combine", b"prefill", b"qk_norm_rope", b"kv_relayout"):
        assert lib.gi_kernel_timing_read(kind, ctypes.byref(ms), ctypes.byref(n)) == 0
        assert (ms.value, n.value) == (0.0, 0)
    assert lib.gi_kernel_timing(0) == 0


def test_layer_harness_built_and_prints_usage():
    # the C++ caller of the ABI; --help exits before touching a GPU
    harness = os.path.join(os.path.dirname(os.path.abspath(__file__)), "..", "ghost-infer_amd", "gi_layer_harness")
    assert os.path.exists(harness), "gi_layer_harness is not built (run __graft_entry__.build())"
    r = subprocess.run([harness, "--help"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0 and "usage: gi_layer_harness" in r.stdout



def test_q4_entry_points_reject_bad_arguments_before_any_launch():
    _fake_pointers_only_without_a_gpu()
    lib = gi_attn.load_library()
    # the 4-bit cache: head size 256 only (the prefill and the operator fix it), 16-byte row strides, scales
    # 4-byte aligned with even strides (the kernels read two scales per 4-byte word)
    ok = dict(q=16, kc=16, vc=16, ks=16, vs=16)

    def decode(ks=16, kv_stride=256, sc_stride=16, sc_head_stride=8):
        return lib.gi_attn_decode_q4(None, ok["q"], 4096, ok["kc"], ok["vc"], ks, 16, kv_stride, 128, sc_stride,
                                     sc_head_stride, 16, 4096, None, 0, 0, None, 0, 1, 16, 2, 0.0625)

    assert decode(kv_stride=200) == -1 and "multiples of 16" in lib.gi_last_error().decode()
    assert decode(ks=18) == -1 and "4-byte aligned" in lib.gi_last_error().decode()
    assert decode(sc_stride=9) == -1 and "strides even" in lib.gi_last_error().decode()
    assert decode(ks=None) == -1 and "scale" in lib.gi_last_error().decode()
    rc = lib.gi_qk_norm_rope_q4(None, 16, None, None, 16, 16, 16, 16, 200, 128, 0, 0, 0, None, 0, 1, 16, 2, 256, 1e4,
                                None, 1, 1e-6)
    assert rc == -1 and "multiples of 16" in lib.gi_last_error().decode()
    rc = lib.gi_qk_norm_rope_q4(None, 16, None, None, 16, 16, None, 16, 256, 128, 0, 0, 0, None, 0, 1, 16, 2, 256, 1e4,
                                None, 1, 1e-6)
    assert rc == -1 and "scale" in lib.gi_last_error().decode()
    rc = lib.gi_hadamard_rows(None, 16, 256, 4, 300)
    assert rc == -1 and "multiple of 256" in lib.gi_last_error().decode()


def test_prefill_workspace_bytes():
    # f16 K and V rows [n_kv][kv_len][hd] (and for int8 f32 scales [n_kv][kv_len]), each region 256-byte aligned;
    # 0 where no widened staging applies (the f16 cache, the f32 kernels' head sizes, the 4-bit cache below 256)
    lib = gi_attn.load_library()

    def a256(x):
        return (x + 255) // 256 * 256

    for kv_len, n_kv, hd in ((8192, 8, 128), (1, 1, 64), (1000, 3, 64), (777, 2, 256)):
        want_i8 = 2 * a256(n_kv * kv_len * hd * 2) + 2 * a256(n_kv * kv_len * 4)
        assert lib.gi_attn_prefill_workspace_bytes(kv_len, n_kv, hd, 1) == want_i8
    assert lib.gi_attn_prefill_workspace_bytes(777, 2, 256, 2) == 2 * a256(2 * 777 * 256 * 2)
    for args in ((100, 2, 128, 0), (100, 2, 96, 1), (100, 2, 128, 2), (0, 2, 128, 1), (100, 0, 128, 1),
                 (100, 2, 72, 1)):
        assert lib.gi_attn_prefill_workspace_bytes(*args) == 0, args


def test_f32_prompts_and_widened_prefill_reject_bad_arguments_before_any_launch():
    _fake_pointers_only_without_a_gpu()
    lib = gi_attn.load_library()
    # gi_attn_prefill_f32: head sizes up to 128 (the reference's attention_prefill)
    rc = lib.gi_attn_prefill_f32(None, 16, 0, 8192, 16, 16, None, None, 0, 512, 256, 0, 0, 16, 0, 4096, 0, 16, 16, 2,
                                 256, 0.0625)
    assert rc == -1 and "up to 128" in lib.gi_last_error().decode()
    # the widened int8 prefill: a workspace is required
    rc = lib.gi_attn_prefill_i8_ws(None, 16, 0, 4096, 16, 16, 16, 16, 1024, 128, 0, 0, 16, 0, 4096, 0, 16, 32, 8, 128,
                                   0.088, None, 0)
    assert rc == -1 and "workspace" in lib.gi_last_error().decode()
