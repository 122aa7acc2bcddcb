"""The cache's edges on the gfx950 path, through the C ABI:

- a device position (graph replay's posp) out of range: the decode kernels clamp it into
  [0, ctx_cap - n_tok] and read no key past ctx_cap; the cache write stores no row outside [0, ctx_cap);
- cache growth (LayerCache::resize, src/cuda.rs:9962-9976, in CTX_STEP = 4096-position steps,
  src/cuda.rs:10410): gi_kv_relayout copies a filled cache into one of a larger capacity; every row is
  bit-identical afterwards and decode over the grown cache gives bit-identical outputs.
"""
import sys

import numpy as np
import pytest
import torch

import gi_attn
from attn_common import assert_close, make_inputs, make_inputs_i8, reference_f64, reference_f64_i8

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


def f16_dev(bits, dev):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(dev).view(torch.float16)


@pytest.mark.parametrize("n_tok", [1, 8])
def test_decode_device_position_edge_and_clamp(gpu, n_tok):
    # the cache holds exactly cap rows; *posp = cap - n_tok is the last valid position, larger or negative ones
    # are clamped to the nearest valid one
    n_heads, n_kv, cap = 32, 4, 2500
    q, k, v = make_inputs(4321 + n_tok, n_tok, cap, n_heads, n_kv)
    qt, kt, vt = torch.from_numpy(q).to(gpu), f16_dev(k, gpu), f16_dev(v, gpu)
    ws = gi_attn.new_workspace(cap, n_tok, n_heads, n_kv, device=gpu)
    posp = torch.zeros(1, dtype=torch.int32, device=gpu)
    edge = cap - n_tok
    for pos, as_pos in ((edge, edge), (edge + 1, edge), (cap + 5000, edge), (1 << 30, edge), (-7, 0)):
        say("decode posp clamp", n_tok, pos)
        posp.fill_(pos)
        out = gi_attn.decode(qt, kt, vt, 0, n_heads, n_kv, workspace=ws, posp=posp, ctx_cap=cap)
        torch.cuda.synchronize()
        assert_close(out.cpu().numpy(), reference_f64(q, k, v, as_pos, n_heads, n_kv), max_abs=2e-5, rel_l2=2e-5,
                     what=f"posp {pos} (as {as_pos})")


def test_decode_i8_device_position_clamp(gpu):
    n_tok, n_heads, n_kv, cap = 1, 32, 4, 2048
    q, k, v, ks, vs = make_inputs_i8(55, n_tok, cap, n_heads, n_kv)
    t = [torch.from_numpy(x).to(gpu) for x in (q, k, v, ks, vs)]
    ws = gi_attn.new_workspace(cap, n_tok, n_heads, n_kv, device=gpu)
    posp = torch.zeros(1, dtype=torch.int32, device=gpu)
    for pos, as_pos in ((cap - 1, cap - 1), (cap + 100, cap - 1)):
        say("decode i8 posp clamp", pos)
        posp.fill_(pos)
        out = gi_attn.decode(t[0], t[1], t[2], 0, n_heads, n_kv, k_scale=t[3], v_scale=t[4], workspace=ws, posp=posp,
                             ctx_cap=cap)
        torch.cuda.synchronize()
        assert_close(out.cpu().numpy(), reference_f64_i8(q, k, v, ks, vs, as_pos, n_heads, n_kv), max_abs=2e-5,
                     rel_l2=2e-5, what=f"i8 posp {pos}")


def test_cache_write_skips_rows_past_capacity(gpu):
    # a device position at or past ctx_cap stores nothing (the q/k rows are still rotated in place)
    n_heads, n_kv, cap, n = 8, 2, 64, 4
    rng = np.random.default_rng(3)
    qkv = torch.from_numpy(rng.standard_normal((n, (n_heads + 2 * n_kv) * 128), dtype=np.float32)).to(gpu)
    kc = torch.full((cap, n_kv, 128), 7.0, dtype=torch.float16, device=gpu)
    vc = torch.full_like(kc, 7.0)
    posp = torch.full((1,), cap - 2, dtype=torch.int32, device=gpu)  # rows cap-2, cap-1 stored, cap, cap+1 not
    say("cache write past capacity")
    gi_attn.qk_norm_rope(qkv, kc, vc, 0, n_heads, n_kv, posp=posp, ctx_cap=cap)
    torch.cuda.synchronize()
    vrows = qkv[:, (n_heads + n_kv) * 128:].reshape(n, n_kv, 128)
    assert torch.equal(vc[cap - 2:], vrows[:2].half())
    assert bool((vc[:cap - 2] == 7.0).all()) and bool((kc[:cap - 2] == 7.0).all())
    # a capacity below the buffer: rows from ctx_cap on are left alone
    kc.fill_(7.0)
    vc.fill_(7.0)
    posp.fill_(30)
    gi_attn.qk_norm_rope(qkv, kc, vc, 0, n_heads, n_kv, posp=posp, ctx_cap=32)
    torch.cuda.synchronize()
    assert bool((vc[32:] == 7.0).all()) and bool((kc[32:] == 7.0).all())
    assert bool((vc[30:32] != 7.0).any())


@pytest.mark.parametrize("i8", [False, True])
def test_cache_growth_relayout_head_major(gpu, i8):
    # a head-major cache filled to `fill` positions grows twice by CTX_STEP; rows and decode outputs are
    # bit-identical before and after
    n_heads, n_kv, cap, fill, step = 32, 4, 4096, 3000, 4096
    if i8:
        q, k, v, ks, vs = make_inputs_i8(17, 1, cap, n_heads, n_kv)
    else:
        q, k, v = make_inputs(17, 1, cap, n_heads, n_kv)

    def head_major(x):
        x = np.ascontiguousarray(x)
        if x.ndim == 2 and x.shape[1] == n_kv:  # scales [cap, n_kv] -> [n_kv, cap]
            return torch.from_numpy(np.ascontiguousarray(x.T)).to(gpu)
        x = x.reshape(cap, n_kv, 128).transpose(1, 0, 2)
        x = np.ascontiguousarray(x)
        return f16_dev(x, gpu) if x.dtype == np.uint16 else torch.from_numpy(x).to(gpu)

    qt = torch.from_numpy(q).to(gpu)
    tensors = [head_major(k), head_major(v)] + ([head_major(ks), head_major(vs)] if i8 else [])
    ws = gi_attn.new_workspace(fill, 1, n_heads, n_kv, device=gpu)

    def run(ts):
        kw = dict(k_scale=ts[2], v_scale=ts[3]) if i8 else {}
        out = gi_attn.decode(qt, ts[0], ts[1], fill - 1, n_heads, n_kv, workspace=ws, kv_layout="head_major", **kw)
        torch.cuda.synchronize()
        return out.cpu().numpy()

    base = run(tensors)
    want = (reference_f64_i8(q, k, v, ks, vs, fill - 1, n_heads, n_kv) if i8
            else reference_f64(q, k, v, fill - 1, n_heads, n_kv))
    assert_close(base, want, max_abs=2e-5, rel_l2=2e-5, what="before growth")
    c = cap
    for g in range(2):
        say("cache growth", "int8" if i8 else "f16", c, "->", c + step)
        grown = []
        for t in tensors:
            shape = (t.shape[0], c + step) + tuple(t.shape[2:])
            d = torch.full(shape, -1 if t.dtype != torch.float16 else 9.0, dtype=t.dtype, device=gpu)
            gi_attn.kv_relayout(t, d, fill, layout="head_major")
            grown.append(d)
        torch.cuda.synchronize()
        for t, d in zip(tensors, grown):
            assert torch.equal(d[:, :fill], t[:, :fill]), "rows differ after growth"
            assert bool((d[:, fill:] == (9.0 if d.dtype == torch.float16 else -1)).all()), "rows past fill written"
        got = run(grown)
        assert np.array_equal(got.view(np.uint32), base.view(np.uint32)), f"decode after growth {g} not bit-identical"
        tensors, c = grown, c + step


def test_cache_growth_relayout_reference_layout(gpu):
    # the reference's [position][n_kv][hd] layout grows by one contiguous copy per buffer
    n_kv, cap, fill = 8, 512, 300
    src = torch.randn((cap, n_kv, 128), device=gpu).half()
    dst = torch.zeros((cap + 4096, n_kv, 128), dtype=torch.float16, device=gpu)
    say("cache growth reference layout")
    gi_attn.kv_relayout(src, dst, fill, layout="reference")
    torch.cuda.synchronize()
    assert torch.equal(dst[:fill], src[:fill]) and bool((dst[fill:] == 0).all())
