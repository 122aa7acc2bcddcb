"""Randomised prefill shapes through every cache format and head size, against float64 attention over the cache's
values on sampled rows (the prefill bar: 2e-3 max-abs, 1e-3 relative L2, since the prefill rounds the scaled
queries and the probabilities to f16 as the reference's attention_prefill_tc does): 16-700 query rows at a prefix
of up to 3000 keys, group sizes 1-8, 1-8 kv heads, f32 or f16 queries and outputs, both cache layouts, seeded so
that a failure names its case and reproduces."""
import sys

import numpy as np
import pytest
import torch

import gi_attn
from attn_common import (assert_close, make_inputs, make_inputs_i8, make_inputs_q4, reference_f64, reference_f64_i8,
                         reference_f64_q4)

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


def cases(fmt, hd, count, seed):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(count):
        n_kv = int(rng.choice([1, 2, 4, 8]))
        G = int(rng.integers(1, 9 if n_kv <= 4 else 5))
        n = int(rng.integers(16, 701))
        pos0 = int(rng.integers(0, 3001))
        qd = str(rng.choice(["f32", "f16"]))
        od = str(rng.choice(["f32", "f16"]))
        layout = str(rng.choice(["reference", "head_major"]))
        out.append((fmt, hd, i, n, pos0, n_kv * G, n_kv, qd, od, layout))
    return out


CASES = (cases("f16", 128, 6, 21) + cases("f16", 256, 6, 22) + cases("i8", 128, 6, 23) + cases("i8", 256, 6, 24)
         + cases("q4", 256, 6, 25) + cases("f16", 64, 4, 26) + cases("i8", 64, 4, 27) + cases("f16", 96, 3, 28)
         + cases("i8", 80, 3, 29))
DT = {"f32": torch.float32, "f16": torch.float16}


def to_layout(t, layout):
    """[ctx, n_kv, ...] -> the layout's tensor (head-major: [n_kv, ctx, ...])."""
    return t.transpose(0, 1).contiguous() if layout == "head_major" else t.contiguous()


@pytest.mark.parametrize("fmt,hd,i,n,pos0,n_heads,n_kv,qd,od,layout", CASES, ids=lambda v: str(v))
def test_random_prefill(gpu, fmt, hd, i, n, pos0, n_heads, n_kv, qd, od, layout):
    say("random prefill", fmt, hd, i, n, pos0, n_heads, n_kv, qd, od, layout)
    seed = 7000 + 131 * i + {"f16": 0, "i8": 1, "q4": 2}[fmt] + hd
    ctx = pos0 + n
    rows = sorted({0, n - 1, *np.random.default_rng(seed).integers(0, n, 4).tolist()})
    if fmt == "f16":
        q, k, v = make_inputs(seed, n, ctx, n_heads, n_kv, hd=hd)
        kt, vt = (to_layout(torch.from_numpy(x.view(np.int16)).to(gpu).view(torch.float16).view(ctx, n_kv, hd), layout)
                  for x in (k, v))
        qt = torch.from_numpy(q).to(gpu).to(DT[qd])
        out = gi_attn.prefill(qt, kt, vt, pos0, n_heads, n_kv, hd=hd, out_dtype=DT[od], kv_layout=layout)

        def want(qr, r):
            return reference_f64(qr, k, v, pos0 + r, n_heads, n_kv, hd=hd)
    elif fmt == "i8":
        q, k, v, ks, vs = make_inputs_i8(seed, n, ctx, n_heads, n_kv, hd=hd)
        kt, vt = (to_layout(torch.from_numpy(x).to(gpu).view(ctx, n_kv, hd), layout) for x in (k, v))
        kst, vst = (to_layout(torch.from_numpy(x).to(gpu), layout) for x in (ks, vs))
        qt = torch.from_numpy(q).to(gpu).to(DT[qd])
        out = gi_attn.prefill(qt, kt, vt, pos0, n_heads, n_kv, hd=hd, out_dtype=DT[od], kv_layout=layout,
                              k_scale=kst, v_scale=vst)

        def want(qr, r):
            return reference_f64_i8(qr, k, v, ks, vs, pos0 + r, n_heads, n_kv, hd=hd)
    else:
        q, kc, vc, ks, vs = make_inputs_q4(seed, n, ctx, n_heads, n_kv)
        c = [to_layout(torch.from_numpy(np.ascontiguousarray(x)).to(gpu).view(ctx, n_kv, 128), layout)
             for x in (kc, vc)]
        s = [to_layout(torch.from_numpy(np.ascontiguousarray(x).view(np.float16)).to(gpu).view(ctx, n_kv, 8), layout)
             for x in (ks, vs)]
        qt = torch.from_numpy(q).to(gpu).to(DT[qd])
        out = gi_attn.prefill_q4(qt, c[0], c[1], s[0], s[1], pos0, n_heads, n_kv, out_dtype=DT[od], kv_layout=layout)

        def want(qr, r):
            return reference_f64_q4(qr, kc, vc, ks, vs, pos0 + r, n_heads, n_kv)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    # the reference sees the queries the kernel was given (f16-rounded when qd is f16)
    qk = qt.float().cpu().numpy()
    for r in rows:
        assert_close(got[r:r + 1], want(qk[r:r + 1], r), what=f"{fmt} hd {hd} case {i} row {r}")
