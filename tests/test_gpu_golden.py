"""The committed golden fixtures (tests/golden/*.npz: seeded inputs and float64 expected outputs, written by
tests/golden/make_golden.py) through the HIP path: the decode / verify cases through gi_attn_decode(_i8, _q4)
and, packed as the reference's qkv rows, through the operator gi_attention(_i8, _q4) (src/cuda.rs:8448-8541);
the prefill cases through gi_attn_prefill(_i8, _q4).

Bar: decode and verify within 2e-5 of float64 (the split path keeps f32 precision), prefill within the
north star's 2e-3 / 1e-3 (it rounds P to f16 as the reference does), and so is decode at head size 256 over the
int8 and 4-bit caches (it rounds Q and P to f16 as the reference's attention_decode_tc256 does)."""
import os
import sys

import numpy as np
import pytest
import torch

import gi_attn
from attn_common import assert_close, split_f64_tol

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
NAMES = sorted(f[:-4] for f in os.listdir(GOLDEN) if f.endswith(".npz"))


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


def load(name, dev):
    z = np.load(os.path.join(GOLDEN, name + ".npz"))
    meta = {k: int(z[k]) for k in ("pos0", "n_heads", "n_kv")}
    meta["hd"] = int(z["hd"]) if "hd" in z.files else 128
    i8 = "ks" in z.files
    q = torch.from_numpy(z["q"]).to(dev)
    if "q4" in z.files:
        nkv = meta["n_kv"]
        k = torch.from_numpy(z["k"]).to(dev).view(-1, nkv, 128)
        v = torch.from_numpy(z["v"]).to(dev).view(-1, nkv, 128)
        sc = dict(k_scale=torch.from_numpy(z["ks"].view(np.float16)).to(dev).view(-1, nkv, 8),
                  v_scale=torch.from_numpy(z["vs"].view(np.float16)).to(dev).view(-1, nkv, 8), q4=True)
    elif i8:
        k, v = torch.from_numpy(z["k"]).to(dev), torch.from_numpy(z["v"]).to(dev)
        sc = dict(k_scale=torch.from_numpy(z["ks"]).to(dev), v_scale=torch.from_numpy(z["vs"]).to(dev))
    else:
        k = torch.from_numpy(z["k"].view(np.int16)).to(dev).view(torch.float16)
        v = torch.from_numpy(z["v"].view(np.int16)).to(dev).view(torch.float16)
        sc = {}
    return z, meta, q, k, v, sc


@pytest.mark.parametrize("name", NAMES)
def test_golden_through_the_hip_path(gpu, name):
    say("golden", name)
    z, m, q, k, v, sc = load(name, gpu)
    n = q.shape[0]
    want = z["out"]
    if sc.pop("q4", False):
        ks, vs = sc["k_scale"], sc["v_scale"]
        if name.startswith("prefill"):
            out = gi_attn.prefill_q4(q, k, v, ks, vs, m["pos0"], m["n_heads"], m["n_kv"], out_dtype=torch.float32)
            torch.cuda.synchronize()
            assert_close(out.cpu().numpy(), want, what=f"{name} prefill")
            return
        out = gi_attn.decode_q4(q, k, v, ks, vs, m["pos0"], m["n_heads"], m["n_kv"])
        torch.cuda.synchronize()
        tol = split_f64_tol("q4", 256)
        assert_close(out.cpu().numpy(), want, *tol, what=f"{name} decode")
        qkv = torch.zeros((n, (m["n_heads"] + 2 * m["n_kv"]) * 256), dtype=torch.float32, device=gpu)
        qkv[:, :m["n_heads"] * 256] = q
        out2 = gi_attn.attention_q4(qkv, k, v, ks, vs, m["pos0"], m["n_heads"], m["n_kv"], exact=True)
        torch.cuda.synchronize()
        assert_close(out2.cpu().numpy(), want, *tol, what=f"{name} operator")
        return
    if name.startswith("prefill"):
        out = gi_attn.prefill(q, k, v, m["pos0"], m["n_heads"], m["n_kv"], hd=m["hd"], out_dtype=torch.float32, **sc)
        torch.cuda.synchronize()
        assert_close(out.cpu().numpy(), want, what=f"{name} prefill")
        return
    out = gi_attn.decode(q, k, v, m["pos0"], m["n_heads"], m["n_kv"], hd=m["hd"], **sc)
    torch.cuda.synchronize()
    tol = split_f64_tol("i8" if sc else "f16", m["hd"])
    assert_close(out.cpu().numpy(), want, *tol, what=f"{name} decode")
    # the operator over the reference's qkv rows [q | k | v] (only q is read: the cache already holds the rows)
    qd, kvd = m["n_heads"] * m["hd"], m["n_kv"] * m["hd"]
    qkv = torch.zeros((n, qd + 2 * kvd), dtype=torch.float32, device=gpu)
    qkv[:, :qd] = q
    out2 = gi_attn.attention(qkv, k, v, m["pos0"], m["n_heads"], m["n_kv"], hd=m["hd"], exact=True, **sc)
    torch.cuda.synchronize()
    assert_close(out2.cpu().numpy(), want, *tol, what=f"{name} operator")
