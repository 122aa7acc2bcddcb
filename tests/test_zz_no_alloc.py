"""gi_attn_decode_noalloc: the decode entry point that allocates nothing (its slice partials live in the code
object's fixed device array) gives the same bits as gi_attn_decode with a caller's workspace, on two calls in a
row (the second smaller), and rejects shapes whose partials exceed the array before launching anything."""
import ctypes
import sys

import numpy as np
import pytest
import torch

import gi_attn

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


def noalloc(q, k, v, pos0, n_heads, n_kv, out, posp=None, ctx_cap=0, hd=128, layout="head_major"):
    kv_stride, kv_head_stride, _ = gi_attn._cache_layout(k, v, n_kv, hd, layout)
    lib = gi_attn.load_library()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    return lib.gi_attn_decode_noalloc(stream, q.data_ptr(), q.stride(0), k.data_ptr(), v.data_ptr(), kv_stride,
                                      kv_head_stride, out.data_ptr(), out.stride(0), pos0,
                                      ctypes.c_void_p(posp.data_ptr()) if posp is not None else None, ctx_cap,
                                      q.shape[0], n_heads, n_kv, hd, 1.0 / np.sqrt(hd))


def test_noalloc_decode_matches_the_workspace_entry_point(gpu):
    gen = torch.Generator(device=gpu)
    gen.manual_seed(2024)
    # config 2's shape, then an 8-token verify block over a smaller cache
    for ctx, n_heads, n_kv, n_tok in ((65536, 32, 4, 1), (3000, 32, 4, 8)):
        say("noalloc decode", ctx, n_heads, n_kv, n_tok)
        k = torch.randn((n_kv, ctx, 128), generator=gen, device=gpu).half()
        v = torch.randn((n_kv, ctx, 128), generator=gen, device=gpu).half()
        q = torch.randn((n_tok, n_heads * 128), generator=gen, device=gpu)
        pos0 = ctx - n_tok
        want = gi_attn.decode(q, k, v, pos0, n_heads, n_kv, kv_layout="head_major")
        out = torch.full_like(want, float("nan"))
        assert noalloc(q, k, v, pos0, n_heads, n_kv, out) == 0, gi_attn.load_library().gi_last_error().decode()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int32), want.view(torch.int32)), "noalloc differs from gi_attn_decode"
    # a device position (graph replay's launch shape) at two positions, the second smaller
    ctx, n_heads, n_kv = 4096, 32, 8
    k = torch.randn((n_kv, ctx, 128), generator=gen, device=gpu).half()
    v = torch.randn((n_kv, ctx, 128), generator=gen, device=gpu).half()
    q = torch.randn((1, n_heads * 128), generator=gen, device=gpu)
    posp = torch.zeros(1, dtype=torch.int32, device=gpu)
    for pos in (4095, 777):
        say("noalloc decode posp", pos)
        posp.fill_(pos)
        want = gi_attn.decode(q, k, v, 0, n_heads, n_kv, posp=posp, ctx_cap=ctx, kv_layout="head_major")
        out = torch.full_like(want, float("nan"))
        assert noalloc(q, k, v, 0, n_heads, n_kv, out, posp=posp, ctx_cap=ctx) == 0
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int32), want.view(torch.int32)), f"noalloc posp {pos} differs"


@pytest.mark.parametrize("hd,n_heads,n_kv", [(64, 9, 3), (256, 16, 2), (80, 32, 32), (96, 12, 4)])
def test_noalloc_other_head_sizes(gpu, hd, n_heads, n_kv):
    # head sizes 64 and 256 on MFMA, 80 and 96 on the f32 kernels: two calls in a row, the second smaller
    gen = torch.Generator(device=gpu)
    gen.manual_seed(hd)
    for ctx, n_tok in ((5000, 3), (700, 1)):
        say("noalloc hd", hd, ctx, n_tok)
        k = torch.randn((n_kv, ctx, hd), generator=gen, device=gpu).half()
        v = torch.randn((n_kv, ctx, hd), generator=gen, device=gpu).half()
        q = torch.randn((n_tok, n_heads * hd), generator=gen, device=gpu)
        pos0 = ctx - n_tok
        want = gi_attn.decode(q, k, v, pos0, n_heads, n_kv, hd=hd, kv_layout="head_major")
        out = torch.full_like(want, float("nan"))
        assert noalloc(q, k, v, pos0, n_heads, n_kv, out, hd=hd) == 0, gi_attn.load_library().gi_last_error().decode()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int32), want.view(torch.int32)), f"noalloc hd {hd} differs"


def test_noalloc_config4_verify_fits(gpu):
    # config 4's verify block (8 tokens at a 32768-key prefix, 32 / 4 heads) fits the array
    gen = torch.Generator(device=gpu)
    gen.manual_seed(7)
    ctx, n_heads, n_kv, n_tok = 32776, 32, 4, 8
    say("noalloc config 4")
    k = torch.randn((n_kv, ctx, 128), generator=gen, device=gpu).half()
    v = torch.randn((n_kv, ctx, 128), generator=gen, device=gpu).half()
    q = torch.randn((n_tok, n_heads * 128), generator=gen, device=gpu)
    want = gi_attn.decode(q, k, v, ctx - n_tok, n_heads, n_kv, kv_layout="head_major")
    out = torch.full_like(want, float("nan"))
    assert noalloc(q, k, v, ctx - n_tok, n_heads, n_kv, out) == 0, gi_attn.load_library().gi_last_error().decode()
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int32), want.view(torch.int32))


REJECT = r"""
import ctypes, os, sys
sys.path.insert(0, os.path.join(sys.argv[1], "ghost-infer_amd"))
import torch, gi_attn
n_tok, n_heads, n_kv, hd, ctx = 8, 32, 4, 128, 32776
chunk, nsplit = gi_attn.decode_plan(ctx, n_tok, n_heads, n_kv, hd)
need = n_tok * n_heads * nsplit * (hd + 4) * 4
assert need > 16 << 20, need
dev = torch.device("cuda:0")
q = torch.zeros((n_tok, n_heads * hd), dtype=torch.float32, device=dev)
k = torch.zeros((n_kv, ctx, hd), dtype=torch.float16, device=dev)
v = torch.zeros_like(k)
out = torch.zeros_like(q)
lib = gi_attn.load_library()
rc = lib.gi_attn_decode_noalloc(None, q.data_ptr(), n_heads * hd, k.data_ptr(), v.data_ptr(), hd, ctx * hd,
                                out.data_ptr(), n_heads * hd, ctx - n_tok, None, 0, n_tok, n_heads, n_kv, hd, 0.088)
torch.cuda.synchronize()
print(rc, lib.gi_last_error().decode(), flush=True)
"""


def test_noalloc_rejects_partials_beyond_the_scratch(gpu, tmp_path):
    # with the default plan no shape's partials exceed the array, so a child process plans for 2048 workgroups
    # (GI_DECODE_TARGET_WGS, read once per process): config 4's verify then needs ~35 MB of partials and must be
    # rejected before any launch. Its buffers are real and sized for the shape, so that a wrong acceptance would
    # launch over valid memory and fail here rather than fault the device.
    import os
    import subprocess
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    say("noalloc rejection (child process)")
    r = subprocess.run([sys.executable, "-c", REJECT, root], capture_output=True, text=True, timeout=120,
                       env=dict(os.environ, GI_DECODE_TARGET_WGS="2048"))
    assert r.returncode == 0, r.stderr[-2000:]
    rc, msg = r.stdout.strip().split(" ", 1)
    assert rc == "-1" and "exceed" in msg, r.stdout
