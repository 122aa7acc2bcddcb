"""Randomised calls of the attention operator (GpuModel::attention's dispatch, src/cuda.rs:8448-8541) over
every cache format: 1-60 tokens of reference-layout qkv rows at a prefix of up to 3000 keys, head sizes 128 and
256, exact or not, against float64 attention over the cache's values. Below 16 tokens, or with `exact`, the
operator takes the split path in launches of at most 15 tokens (the split path's bar, 2e-5; at head size 256 over
the int8 and 4-bit caches, whose split path rounds Q and P to f16 as the reference does, the north star's); from 16
tokens it
takes the prefill kernel (the prefill bar, 2e-3 max-abs and 1e-3 relative L2). With bit 1 of `exact` (the
reference's GHOST_INFER_NO_TC_ATT) every batch computes in f32 precision (the 2e-5 bar). Seeded, so that a failure
names its case and reproduces."""
import sys

import numpy as np
import pytest
import torch

import gi_attn
from attn_common import (assert_close, make_inputs, make_inputs_i8, make_inputs_q4, reference_f64, reference_f64_i8,
                         reference_f64_q4, split_f64_tol)

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


def cases(fmt, count, seed):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(count):
        n_kv = int(rng.choice([1, 2, 4, 8]))
        G = int(rng.integers(1, 9))
        n = int(rng.choice([int(rng.integers(1, 16)), int(rng.integers(16, 61))]))
        pos0 = int(rng.integers(0, 3001))
        hd = 256 if fmt == "q4" else int(rng.choice([64, 96, 128, 256]))
        exact = bool(rng.integers(0, 2))
        out.append((fmt, i, n, pos0, n_kv * G, n_kv, hd, exact))
    return out


CASES = cases("f16", 8, 31) + cases("i8", 8, 32) + cases("q4", 6, 33)


@pytest.mark.parametrize("fmt,i,n,pos0,n_heads,n_kv,hd,exact", CASES, ids=lambda v: str(v))
def test_random_operator(gpu, fmt, i, n, pos0, n_heads, n_kv, hd, exact):
    say("random operator", fmt, i, n, pos0, n_heads, n_kv, hd, exact)
    seed = 9000 + 71 * i + {"f16": 0, "i8": 1, "q4": 2}[fmt]
    ctx = pos0 + n
    # the operator reads only the q part of each [q | k | v] row: the cache already holds the batch's K/V
    row = n_heads * hd + 2 * n_kv * hd
    qkv = np.random.default_rng(seed + 10).standard_normal((n, row), dtype=np.float32)
    qt = torch.from_numpy(qkv).to(gpu)
    q = np.ascontiguousarray(qkv[:, :n_heads * hd])
    if fmt == "f16":
        _, k, v = make_inputs(seed, 1, ctx, n_heads, n_kv, hd=hd)
        kt, vt = (torch.from_numpy(x.view(np.int16)).to(gpu).view(torch.float16).view(ctx, n_kv, hd) for x in (k, v))
        out = gi_attn.attention(qt, kt, vt, pos0, n_heads, n_kv, hd=hd, exact=exact)
        want = reference_f64(q, k, v, pos0, n_heads, n_kv, hd=hd)
    elif fmt == "i8":
        _, k, v, ks, vs = make_inputs_i8(seed, 1, ctx, n_heads, n_kv, hd=hd)
        kt, vt = (torch.from_numpy(x).to(gpu).view(ctx, n_kv, hd) for x in (k, v))
        kst, vst = (torch.from_numpy(x).to(gpu) for x in (ks, vs))
        out = gi_attn.attention(qt, kt, vt, pos0, n_heads, n_kv, hd=hd, exact=exact, k_scale=kst, v_scale=vst)
        want = reference_f64_i8(q, k, v, ks, vs, pos0, n_heads, n_kv, hd=hd)
    else:
        _, kc, vc, ks, vs = make_inputs_q4(seed, 1, ctx, n_heads, n_kv)
        c = [torch.from_numpy(np.ascontiguousarray(x)).to(gpu).view(ctx, n_kv, 128) for x in (kc, vc)]
        s = [torch.from_numpy(np.ascontiguousarray(x).view(np.float16)).to(gpu).view(ctx, n_kv, 8) for x in (ks, vs)]
        out = gi_attn.attention_q4(qt, c[0], c[1], s[0], s[1], pos0, n_heads, n_kv, exact=exact)
        # the queries are taken as already rotated (as qk_norm_rope_q4 leaves them), and the operator returns the
        # rotated rows, which the layer turns back with hadamard_rows
        want = reference_f64_q4(q, kc, vc, ks, vs, pos0, n_heads, n_kv)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    split = n < 16 or exact
    tol = split_f64_tol(fmt, hd) if split else (2e-3, 1e-3)
    assert_close(got, want, max_abs=tol[0], rel_l2=tol[1], what=f"{fmt} case {i} ({'split' if split else 'prefill'})")


NO_TC_CASES = [c + (True,) for c in cases("f16", 6, 34) + cases("i8", 6, 35)]


@pytest.mark.parametrize("fmt,i,n,pos0,n_heads,n_kv,hd,exact,no_tc", NO_TC_CASES, ids=lambda v: str(v))
def test_random_operator_no_tc(gpu, fmt, i, n, pos0, n_heads, n_kv, hd, exact, no_tc):
    # bit 1 of exact (GHOST_INFER_NO_TC_ATT): every batch in f32 precision (prompts up to head size 128 on the f32
    # prefill, the rest on the split path, head size 256 over int8 without the tc256 roundings): the 2e-5 bar
    say("random operator no_tc", fmt, i, n, pos0, n_heads, n_kv, hd, exact)
    seed = 9500 + 71 * i + {"f16": 0, "i8": 1}[fmt]
    ctx = pos0 + n
    row = n_heads * hd + 2 * n_kv * hd
    qkv = np.random.default_rng(seed + 10).standard_normal((n, row), dtype=np.float32)
    qt = torch.from_numpy(qkv).to(gpu)
    q = np.ascontiguousarray(qkv[:, :n_heads * hd])
    if fmt == "f16":
        _, k, v = make_inputs(seed, 1, ctx, n_heads, n_kv, hd=hd)
        kt, vt = (torch.from_numpy(x.view(np.int16)).to(gpu).view(torch.float16).view(ctx, n_kv, hd) for x in (k, v))
        out = gi_attn.attention(qt, kt, vt, pos0, n_heads, n_kv, hd=hd, exact=exact, no_tc=no_tc)
        want = reference_f64(q, k, v, pos0, n_heads, n_kv, hd=hd)
    else:
        _, k, v, ks, vs = make_inputs_i8(seed, 1, ctx, n_heads, n_kv, hd=hd)
        kt, vt = (torch.from_numpy(x).to(gpu).view(ctx, n_kv, hd) for x in (k, v))
        kst, vst = (torch.from_numpy(x).to(gpu) for x in (ks, vs))
        out = gi_attn.attention(qt, kt, vt, pos0, n_heads, n_kv, hd=hd, exact=exact, k_scale=kst, v_scale=vst,
                                no_tc=no_tc)
        want = reference_f64_i8(q, k, v, ks, vs, pos0, n_heads, n_kv, hd=hd)
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), want, *split_f64_tol("f16", hd), what=f"{fmt} case {i} no_tc")
