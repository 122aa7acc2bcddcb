"""Parity of the f32 kernels (gi_attn_f32.hip) through the C ABI: head sizes the MFMA kernels do not take, the
multiples of 16 up to 112 other than 64 (Phi-2-style 80, Phi-3-style 96, and 16, 32, 48, 112), over the f16 and
the int8 cache. They are the reference's f32 fallback cases: attention_partial for decode (src/cuda.rs:1866-1932)
and attention_prefill for prompts (src/cuda.rs:1934-2041).

Bar: decode and prefill within 2e-5 of float64 attention over the cache's values (both compute in f32, with no f16
rounding of Q or P), and within the north star's bar of the oracle's Model::attention (src/model.rs:1320-1409)."""
import sys

import numpy as np
import pytest
import torch

import gi_attn
import gi_oracle as O
from attn_common import SPLIT_F64_TOL, assert_close, make_inputs, make_inputs_i8, reference_f64, reference_f64_i8

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


def f16_dev(x, dev):
    return torch.from_numpy(np.ascontiguousarray(x).view(np.int16)).to(dev).view(torch.float16)


def deq(c, sc, n_kv, hd):
    return (c.reshape(c.shape[0], n_kv, hd).astype(np.float32) * sc[:, :, None]).reshape(c.shape[0], -1)


DECODE_SHAPES = [
    # (n_tok, pos0, n_heads, n_kv, hd): one slice and several (256-key tiles inside a slice), MHA and GQA
    (1, 0, 32, 32, 80),
    (1, 300, 32, 32, 80),
    (1, 4095, 32, 32, 96),
    (3, 2000, 32, 8, 96),
    (8, 700, 12, 4, 112),
    (15, 513, 8, 1, 48),
    (1, 20000, 16, 4, 32),
    (2, 77, 4, 2, 16),
    (15, 0, 6, 2, 112),     # every token's span inside the first tile
    (4, 65535, 8, 8, 80),   # many slices, a span ending one key short of a tile
]


@pytest.mark.parametrize("n_tok,pos0,n_heads,n_kv,hd", DECODE_SHAPES)
@pytest.mark.parametrize("i8", [False, True])
def test_decode_f32_kernels(gpu, n_tok, pos0, n_heads, n_kv, hd, i8):
    say("decode f32", n_tok, pos0, n_heads, n_kv, hd, i8)
    if i8:
        q, k, v, ks, vs = make_inputs_i8(5100 + pos0 + hd, n_tok, pos0 + n_tok, n_heads, n_kv, hd=hd)
        t = [torch.from_numpy(x).to(gpu) for x in (q, k, v, ks, vs)]
        out = gi_attn.decode(t[0], t[1], t[2], pos0, n_heads, n_kv, hd=hd, k_scale=t[3], v_scale=t[4])
        want = reference_f64_i8(q, k, v, ks, vs, pos0, n_heads, n_kv, hd=hd)
        orc = O.attention(q, deq(k, ks, n_kv, hd), deq(v, vs, n_kv, hd), pos0, n_heads, n_kv, hd=hd)
    else:
        q, k, v = make_inputs(5000 + pos0 + hd, n_tok, pos0 + n_tok, n_heads, n_kv, hd=hd)
        out = gi_attn.decode(torch.from_numpy(q).to(gpu), f16_dev(k, gpu), f16_dev(v, gpu), pos0, n_heads, n_kv, hd=hd)
        want = reference_f64(q, k, v, pos0, n_heads, n_kv, hd=hd)
        orc = O.attention(q, k, v, pos0, n_heads, n_kv, hd=hd)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert_close(got, orc, what="decode f32 vs oracle (Model::attention)")
    assert_close(got, want, *SPLIT_F64_TOL, what="decode f32 vs f64")


def test_decode_f32_graph_replay(gpu):
    # a device position with the launch sized for ctx_cap, captured once and replayed at several positions
    n_tok, n_heads, n_kv, hd, cap = 2, 32, 32, 80, 2000
    q, k, v = make_inputs(5200, n_tok, cap, n_heads, n_kv, hd=hd)
    qt, kt, vt = torch.from_numpy(q).to(gpu), f16_dev(k, gpu), f16_dev(v, gpu)
    ws = gi_attn.new_workspace(cap, n_tok, n_heads, n_kv, hd=hd, device=gpu)
    posp = torch.zeros(1, dtype=torch.int32, device=gpu)
    out = torch.zeros((n_tok, n_heads * hd), dtype=torch.float32, device=gpu)
    kw = dict(hd=hd, out=out, workspace=ws, posp=posp, ctx_cap=cap)
    gi_attn.decode(qt, kt, vt, 0, n_heads, n_kv, **kw)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        gi_attn.decode(qt, kt, vt, 0, n_heads, n_kv, **kw)
    for pos in (cap - n_tok, 300, 0):
        say("decode f32 graph replay", pos)
        posp.fill_(pos)
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert_close(out.cpu().numpy(), reference_f64(q, k, v, pos, n_heads, n_kv, hd=hd), *SPLIT_F64_TOL,
                     what=f"f32 replay at {pos}")


PREFILL_SHAPES = [
    # (n, pos0, n_heads, n_kv, hd, q dtype, out dtype, layout): one and several 32-row tiles, chunks at a prefix
    (16, 0, 32, 32, 80, np.float32, torch.float32, "reference"),
    (100, 0, 32, 32, 96, np.float16, torch.float32, "head_major"),
    (257, 3, 12, 4, 112, np.float32, torch.float16, "reference"),
    (64, 500, 8, 1, 48, np.float16, torch.float32, "reference"),
    (33, 0, 4, 2, 16, np.float32, torch.float32, "head_major"),
    (600, 0, 16, 4, 32, np.float32, torch.float32, "reference"),
    # one row, a few rows and the 128-row workgroup's edges, after a prefix (a chunk of a longer prompt)
    (1, 0, 8, 8, 80, np.float32, torch.float32, "reference"),
    (1, 700, 8, 2, 96, np.float16, torch.float32, "head_major"),
    (5, 61, 6, 3, 48, np.float32, torch.float32, "reference"),
    (127, 1, 4, 4, 112, np.float32, torch.float32, "reference"),
    (129, 200, 4, 1, 80, np.float32, torch.float32, "head_major"),
    (300, 4000, 2, 2, 16, np.float16, torch.float16, "reference"),
]


@pytest.mark.parametrize("n,pos0,n_heads,n_kv,hd,qd,od,layout", PREFILL_SHAPES)
@pytest.mark.parametrize("i8", [False, True])
def test_prefill_f32_kernels(gpu, n, pos0, n_heads, n_kv, hd, qd, od, layout, i8):
    say("prefill f32", n, pos0, n_heads, n_kv, hd, qd.__name__, od, layout, i8)
    if i8:
        q, k, v, ks, vs = make_inputs_i8(5300 + n + pos0, n, pos0 + n, n_heads, n_kv, hd=hd)
        q = q.astype(qd)
        kd = [np.ascontiguousarray(x) for x in (k, v, ks, vs)]
        if layout == "head_major":
            kd = [np.ascontiguousarray(x.reshape(x.shape[0], n_kv, hd).transpose(1, 0, 2)) for x in kd[:2]] + \
                 [np.ascontiguousarray(x.T) for x in kd[2:]]
        t = [torch.from_numpy(x).to(gpu) for x in kd]
        out = gi_attn.prefill(torch.from_numpy(q).to(gpu), t[0], t[1], pos0, n_heads, n_kv, hd=hd, out_dtype=od,
                              kv_layout=layout, k_scale=t[2], v_scale=t[3])
        want = reference_f64_i8(q.astype(np.float32), k, v, ks, vs, pos0, n_heads, n_kv, hd=hd)
    else:
        q, k, v = make_inputs(5400 + n + pos0, n, pos0 + n, n_heads, n_kv, hd=hd, q_dtype=qd)
        kt, vt = f16_dev(k, gpu), f16_dev(v, gpu)
        if layout == "head_major":
            kt = kt.view(-1, n_kv, hd).transpose(0, 1).contiguous()
            vt = vt.view(-1, n_kv, hd).transpose(0, 1).contiguous()
        out = gi_attn.prefill(torch.from_numpy(q).to(gpu), kt, vt, pos0, n_heads, n_kv, hd=hd, out_dtype=od,
                              kv_layout=layout)
        want = reference_f64(q.astype(np.float32), k, v, pos0, n_heads, n_kv, hd=hd)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    # f32 throughout; an f16 output adds its own rounding (2^-11 relative)
    tol = SPLIT_F64_TOL if od == torch.float32 else (2e-3, 1e-3)
    assert_close(got, want, *tol, what="prefill f32 vs f64")


@pytest.mark.parametrize("n,pos0,exact,i8", [(1, 99, False, False), (20, 0, False, False), (40, 17, True, False),
                                             (20, 0, False, True), (8, 300, True, True)])
def test_attention_operator_f32_head_size(gpu, n, pos0, exact, i8):
    # Phi-3-shaped heads (32 heads of 96, no grouping) over the reference's qkv rows
    say("operator f32", n, pos0, exact, i8)
    n_heads, n_kv, hd = 32, 32, 96
    row = (n_heads + 2 * n_kv) * hd
    qkv = np.random.default_rng(597 + n).standard_normal((n, row), dtype=np.float32)
    qkv_t = torch.from_numpy(qkv).to(gpu)
    q = np.ascontiguousarray(qkv[:, :n_heads * hd])
    if i8:
        _, k, v, ks, vs = make_inputs_i8(598 + n, 1, pos0 + n, n_heads, n_kv, hd=hd)
        t = [torch.from_numpy(x).to(gpu) for x in (k, v, ks, vs)]
        out = gi_attn.attention(qkv_t, t[0].view(-1, n_kv, hd), t[1].view(-1, n_kv, hd), pos0, n_heads, n_kv, hd=hd,
                                exact=exact, k_scale=t[2], v_scale=t[3])
        want = reference_f64_i8(q, k, v, ks, vs, pos0, n_heads, n_kv, hd=hd)
    else:
        _, k, v = make_inputs(598 + n, 1, pos0 + n, n_heads, n_kv, hd=hd)
        out = gi_attn.attention(qkv_t, f16_dev(k, gpu), f16_dev(v, gpu), pos0, n_heads, n_kv, hd=hd, exact=exact)
        want = reference_f64(q, k, v, pos0, n_heads, n_kv, hd=hd)
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), want, *SPLIT_F64_TOL, what="operator f32 head size vs f64")


F32_PROMPT_SHAPES = [
    # (n, pos0, n_heads, n_kv, hd, layout, int8): the reference's attention_prefill with its tensor-core prefill off
    (16, 0, 8, 2, 128, "reference", False),
    (300, 0, 32, 8, 128, "head_major", False),
    (129, 700, 16, 4, 128, "reference", True),
    (200, 0, 9, 3, 64, "head_major", False),
    (64, 3000, 8, 8, 64, "reference", True),
]


@pytest.mark.parametrize("n,pos0,n_heads,n_kv,hd,layout,i8", F32_PROMPT_SHAPES)
def test_prefill_f32_prompts_at_mfma_head_sizes(gpu, n, pos0, n_heads, n_kv, hd, layout, i8):
    say("prefill f32 prompts", n, pos0, n_heads, n_kv, hd, layout, i8)
    if i8:
        q, k, v, ks, vs = make_inputs_i8(5500 + n + pos0, n, pos0 + n, n_heads, n_kv, hd=hd)
        kd = [np.ascontiguousarray(x) for x in (k, v, ks, vs)]
        if layout == "head_major":
            kd = [np.ascontiguousarray(x.reshape(x.shape[0], n_kv, hd).transpose(1, 0, 2)) for x in kd[:2]] + \
                 [np.ascontiguousarray(x.T) for x in kd[2:]]
        t = [torch.from_numpy(x).to(gpu) for x in kd]
        out = gi_attn.prefill(torch.from_numpy(q).to(gpu), t[0], t[1], pos0, n_heads, n_kv, hd=hd,
                              out_dtype=torch.float32, kv_layout=layout, k_scale=t[2], v_scale=t[3], f32=True)
        want = reference_f64_i8(q, k, v, ks, vs, pos0, n_heads, n_kv, hd=hd)
    else:
        q, k, v = make_inputs(5600 + n + pos0, n, pos0 + n, n_heads, n_kv, hd=hd)
        kt, vt = f16_dev(k, gpu), f16_dev(v, gpu)
        if layout == "head_major":
            kt = kt.view(-1, n_kv, hd).transpose(0, 1).contiguous()
            vt = vt.view(-1, n_kv, hd).transpose(0, 1).contiguous()
        out = gi_attn.prefill(torch.from_numpy(q).to(gpu), kt, vt, pos0, n_heads, n_kv, hd=hd, out_dtype=torch.float32,
                              kv_layout=layout, f32=True)
        want = reference_f64(q, k, v, pos0, n_heads, n_kv, hd=hd)
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), want, *SPLIT_F64_TOL, what="f32 prompts vs f64")


@pytest.mark.parametrize("hd,i8,n", [(128, False, 40), (128, True, 40), (64, False, 40), (256, False, 40),
                                    (256, True, 40), (256, True, 5), (256, True, 12)])
def test_operator_f32_prompts_matches_the_split_path(gpu, hd, i8, n):
    # bit 1 of exact (GHOST_INFER_NO_TC_ATT): prompts in f32; head size 256 has no such kernel and takes the split path,
    # over the int8 cache in f32 precision (attention_partial_gqa's hd-256 branch) instead of the tc256 roundings
    pos0 = 90
    n_heads, n_kv = (16, 2) if hd == 256 else (8, 2)
    say("operator f32 prompts", hd, i8, n)
    row = (n_heads + 2 * n_kv) * hd
    qkv = np.random.default_rng(777 + hd).standard_normal((n, row), dtype=np.float32)
    qkv_t = torch.from_numpy(qkv).to(gpu)
    q = np.ascontiguousarray(qkv[:, :n_heads * hd])
    if i8:
        _, k, v, ks, vs = make_inputs_i8(778 + hd, 1, pos0 + n, n_heads, n_kv, hd=hd)
        t = [torch.from_numpy(x).to(gpu) for x in (k, v, ks, vs)]
        kw = dict(hd=hd, k_scale=t[2], v_scale=t[3])
        kc, vc = t[0].view(-1, n_kv, hd), t[1].view(-1, n_kv, hd)
        want = reference_f64_i8(q, k, v, ks, vs, pos0, n_heads, n_kv, hd=hd)
    else:
        _, k, v = make_inputs(778 + hd, 1, pos0 + n, n_heads, n_kv, hd=hd)
        kw = dict(hd=hd)
        kc, vc = f16_dev(k, gpu), f16_dev(v, gpu)
        want = reference_f64(q, k, v, pos0, n_heads, n_kv, hd=hd)
    a = gi_attn.attention(qkv_t, kc, vc, pos0, n_heads, n_kv, no_tc=True, **kw)
    b = gi_attn.attention(qkv_t, kc, vc, pos0, n_heads, n_kv, exact=True, **kw)
    torch.cuda.synchronize()
    assert_close(a.cpu().numpy(), want, *SPLIT_F64_TOL, what="f32 prompts vs f64")
    # (exact = 1 at head size 256 over the int8 cache keeps the tc256 roundings: the parity bar between the two)
    ab_tol = (2e-3, 1e-3) if hd == 256 and i8 else SPLIT_F64_TOL
    assert_close(a.cpu().numpy(), b.cpu().numpy(), *ab_tol, what="f32 prompts vs the split path")


@pytest.mark.parametrize("hd,i8", [(128, False), (256, True)])
def test_operator_verify_with_no_tc(gpu, hd, i8):
    # bits 0 and 1 of exact: a verify batch under GHOST_INFER_NO_TC_ATT stays on the split path (every token a
    # decode step, as s.exact does), in f32 precision at head size 256 over the int8 cache as well
    n, pos0 = 40, 90
    n_heads, n_kv = (16, 2) if hd == 256 else (8, 2)
    say("operator verify no_tc", hd, i8)
    row = (n_heads + 2 * n_kv) * hd
    qkv = np.random.default_rng(888 + hd).standard_normal((n, row), dtype=np.float32)
    qkv_t = torch.from_numpy(qkv).to(gpu)
    q = np.ascontiguousarray(qkv[:, :n_heads * hd])
    if i8:
        _, k, v, ks, vs = make_inputs_i8(889 + hd, 1, pos0 + n, n_heads, n_kv, hd=hd)
        t = [torch.from_numpy(x).to(gpu) for x in (k, v, ks, vs)]
        kw = dict(hd=hd, k_scale=t[2], v_scale=t[3])
        kc, vc = t[0].view(-1, n_kv, hd), t[1].view(-1, n_kv, hd)
        want = reference_f64_i8(q, k, v, ks, vs, pos0, n_heads, n_kv, hd=hd)
    else:
        _, k, v = make_inputs(889 + hd, 1, pos0 + n, n_heads, n_kv, hd=hd)
        kw = dict(hd=hd)
        kc, vc = f16_dev(k, gpu), f16_dev(v, gpu)
        want = reference_f64(q, k, v, pos0, n_heads, n_kv, hd=hd)
    a = gi_attn.attention(qkv_t, kc, vc, pos0, n_heads, n_kv, exact=True, no_tc=True, **kw)
    torch.cuda.synchronize()
    assert_close(a.cpu().numpy(), want, *SPLIT_F64_TOL, what="verify under no_tc vs f64")
    if not i8:  # the split path itself: the same kernels as exact alone, bit for bit
        b = gi_attn.attention(qkv_t, kc, vc, pos0, n_heads, n_kv, exact=True, **kw)
        torch.cuda.synchronize()
        assert torch.equal(a, b)
