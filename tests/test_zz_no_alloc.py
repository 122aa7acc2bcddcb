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


def test_noalloc_rejects_partials_beyond_the_scratch(gpu):
    # 15 tokens x 128 heads of size 256 on one kv head over a million keys: ~34 MB of partials
    lib = gi_attn.load_library()
    rc = lib.gi_attn_decode_noalloc(None, 16, 128 * 256, 16, 16, 256, 256 * (1 << 20), 16, 128 * 256, (1 << 20) - 15,
                                    None, 0, 15, 128, 1, 256, 0.0625)
    assert rc == -1 and "exceed" in lib.gi_last_error().decode()
