"""Randomised decode shapes through every cache format and head size, against float64 attention over the
cache's values (the split path's bar: 2e-5 max-abs and relative L2; head size 256 over the int8 and 4-bit caches,
which round Q and P to f16 as the reference's attention_decode_tc256 does, the north star's bar) and, for those, the
oracle's restatement of attention_decode_tc256 (REF_ORACLE_TOL): token counts 1-15, spans up to 6000 keys, group
sizes 1-8 and 1-8 kv heads, seeded so that a failure names its case and reproduces."""
import sys

import numpy as np
import pytest
import torch

import gi_attn
import gi_oracle as O
from attn_common import (REF_ORACLE_TOL, assert_close, make_inputs, make_inputs_i8, make_inputs_q4, reference_f64,
                         reference_f64_i8, reference_f64_q4, split_f64_tol)

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


def cases(fmt, count=12, seed=0):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(count):
        n_kv = int(rng.choice([1, 2, 4, 8]))
        G = int(rng.integers(1, 9))
        n_tok = int(rng.integers(1, 16))
        pos0 = int(rng.integers(0, 6000))
        hd = 256 if fmt == "q4" else int(rng.choice([128, 256]))
        out.append((fmt, i, n_tok, pos0, n_kv * G, n_kv, hd))
    return out


def cases_hd(fmt, hds, count, seed):
    """Cases at head sizes beyond 128 and 256: 64 (the MFMA kernels) and the f32 kernels' multiples of 16."""
    rng = np.random.default_rng(seed)
    out = []
    for i in range(count):
        n_kv = int(rng.choice([1, 2, 4, 8]))
        out.append((fmt, 100 + i, int(rng.integers(1, 16)), int(rng.integers(0, 6000)), n_kv * int(rng.integers(1, 9)),
                    n_kv, int(rng.choice(hds))))
    return out


CASES = (cases("f16", seed=11) + cases("i8", seed=12) + cases("q4", seed=13) + cases_hd("f16", [64], 6, 14)
         + cases_hd("i8", [64], 6, 15) + cases_hd("f16", [16, 32, 48, 80, 96, 112], 6, 16)
         + cases_hd("i8", [32, 80, 96, 112], 4, 17))


@pytest.mark.parametrize("fmt,i,n_tok,pos0,n_heads,n_kv,hd", CASES, ids=lambda v: str(v))
def test_random_decode(gpu, fmt, i, n_tok, pos0, n_heads, n_kv, hd):
    say("random decode", fmt, i, n_tok, pos0, n_heads, n_kv, hd)
    seed = 3000 + 97 * i + {"f16": 0, "i8": 1, "q4": 2}[fmt]
    if fmt == "f16":
        q, k, v = make_inputs(seed, n_tok, pos0 + n_tok, n_heads, n_kv, hd=hd)
        kt = torch.from_numpy(k.view(np.int16)).to(gpu).view(torch.float16)
        vt = torch.from_numpy(v.view(np.int16)).to(gpu).view(torch.float16)
        out = gi_attn.decode(torch.from_numpy(q).to(gpu), kt, vt, pos0, n_heads, n_kv, hd=hd)
        want = reference_f64(q, k, v, pos0, n_heads, n_kv, hd=hd)
    elif fmt == "i8":
        q, k, v, ks, vs = make_inputs_i8(seed, n_tok, pos0 + n_tok, n_heads, n_kv, hd=hd)
        t = [torch.from_numpy(x).to(gpu) for x in (q, k, v, ks, vs)]
        out = gi_attn.decode(t[0], t[1], t[2], pos0, n_heads, n_kv, hd=hd, k_scale=t[3], v_scale=t[4])
        want = reference_f64_i8(q, k, v, ks, vs, pos0, n_heads, n_kv, hd=hd)
        ref = O.decode_tc256_i8(q, k, v, ks, vs, pos0, n_heads, n_kv) if hd == 256 else None
    else:
        q, kc, vc, ks, vs = make_inputs_q4(seed, n_tok, pos0 + n_tok, n_heads, n_kv)
        c = [torch.from_numpy(np.ascontiguousarray(x)).to(gpu).view(-1, n_kv, 128) for x in (kc, vc)]
        s = [torch.from_numpy(np.ascontiguousarray(x).view(np.float16)).to(gpu).view(-1, n_kv, 8) for x in (ks, vs)]
        out = gi_attn.decode_q4(torch.from_numpy(q).to(gpu), c[0], c[1], s[0], s[1], pos0, n_heads, n_kv)
        want = reference_f64_q4(q, kc, vc, ks, vs, pos0, n_heads, n_kv)
        ref = O.decode_tc256_q4(q, kc, vc, ks, vs, pos0, n_heads, n_kv)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    if fmt != "f16" and hd == 256:
        assert_close(got, ref, *REF_ORACLE_TOL, what=f"{fmt} case {i} vs oracle")
    assert_close(got, want, *split_f64_tol(fmt, hd), what=f"{fmt} case {i}")
