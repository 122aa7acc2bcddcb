"""Scores that keep rising along the sequence, so that every kernel's running maximum moves many times: the decode
kernels' lazy rescale (a slice keeps its reference maximum until a score passes it by 2^8 in p) and the prefill's
(PF_RESCALE_LOG2), and the f32 kernels' exact online softmax. The queries and keys share a direction whose key
component ramps up with the position: for the decode 80 log2 units over 1024 keys (slices of 128 keys: each sees its
maximum move by ~10 (head size 256: slices of 64, ~5), and the slices' maxima differ by up to 80 in the merge), for the prefill 30 over 1000 (a row's
reference maximum moves every ~270 keys). Bars: the split decode within 2e-5 of float64 (head size 256 over the int8
cache: attention_decode_tc256's roundings, the parity bar); the prefill, whose Q and P are rounded to f16 as the
reference's attention_prefill_tc does, against the oracle's restatement of those roundings at the parity bar (an
f16-rounded Q moves scores of this size by more than the float64 bar allows)."""
import sys

import numpy as np
import pytest
import torch

import gi_attn
import gi_oracle as O
from attn_common import REF_ORACLE_TOL, SPLIT_F64_TOL, assert_close, reference_f64, reference_f64_i8, split_f64_tol

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


def ramp_inputs(seed, n_tok, ctx, n_heads, n_kv, hd, i8=False, log2_span=30.0):
    """q [n_tok, n_heads*hd] f32; K/V rows [ctx, n_kv*hd] (f16 bits, or int8 codes with f32 scales [ctx, n_kv] as
    kv_store quantises them): N(0,1) plus, along e = ones/sqrt(hd) in every head, A for the queries and a ramp
    0..B over the positions for the keys, with A*B/sqrt(hd)*log2(e) = log2_span."""
    rng = np.random.default_rng(seed)
    e = np.ones(hd, dtype=np.float64) / np.sqrt(hd)
    ab = log2_span * np.sqrt(hd) / np.log2(np.e)
    A = np.sqrt(ab / 2.0)
    B = ab / A
    q = rng.standard_normal((n_tok, n_heads, hd)) + A * e
    k = rng.standard_normal((ctx, n_kv, hd)) + (B * np.arange(ctx) / max(ctx - 1, 1))[:, None, None] * e
    v = rng.standard_normal((ctx, n_kv, hd))
    q = q.reshape(n_tok, -1).astype(np.float32)
    if i8:
        kc, ks = O.kv_quant_i8(k.astype(np.float32))
        vc, vs = O.kv_quant_i8(v.astype(np.float32))
        return q, kc.reshape(ctx, -1), vc.reshape(ctx, -1), ks, vs
    return q, k.reshape(ctx, -1).astype(np.float16).view(np.uint16), v.reshape(ctx, -1).astype(np.float16).view(np.uint16)


def f16_dev(x, dev):
    return torch.from_numpy(np.ascontiguousarray(x).view(np.int16)).to(dev).view(torch.float16)


@pytest.mark.parametrize("hd", [64, 128, 256, 80])
@pytest.mark.parametrize("n_tok", [1, 8])
def test_decode_rising_scores_f16(gpu, hd, n_tok):
    ctx, n_heads, n_kv = 1024, 8, 2
    say("rescale decode f16", hd, n_tok)
    q, k, v = ramp_inputs(7000 + hd + n_tok, n_tok, ctx, n_heads, n_kv, hd, log2_span=80.0)
    pos0 = ctx - n_tok
    out = gi_attn.decode(torch.from_numpy(q).to(gpu), f16_dev(k, gpu), f16_dev(v, gpu), pos0, n_heads, n_kv, hd=hd)
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), reference_f64(q, k, v, pos0, n_heads, n_kv, hd=hd), *SPLIT_F64_TOL,
                 what=f"rising scores, decode hd {hd}")


@pytest.mark.parametrize("hd", [64, 128, 256])
@pytest.mark.parametrize("n_tok", [1, 8])
def test_decode_rising_scores_i8(gpu, hd, n_tok):
    ctx, n_heads, n_kv = 1024, 8, 2
    say("rescale decode i8", hd, n_tok)
    q, kc, vc, ks, vs = ramp_inputs(7100 + hd + n_tok, n_tok, ctx, n_heads, n_kv, hd, i8=True, log2_span=80.0)
    pos0 = ctx - n_tok
    t = [torch.from_numpy(x).to(gpu) for x in (q, kc, vc, ks, vs)]
    out = gi_attn.decode(t[0], t[1], t[2], pos0, n_heads, n_kv, hd=hd, k_scale=t[3], v_scale=t[4])
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert_close(got, reference_f64_i8(q, kc, vc, ks, vs, pos0, n_heads, n_kv, hd=hd), *split_f64_tol("i8", hd),
                 what=f"rising scores, int8 decode hd {hd}")
    if hd == 256:  # the tc256 roundings: against the oracle's restatement too
        assert_close(got, O.decode_tc256_i8(q, kc, vc, ks, vs, pos0, n_heads, n_kv), *REF_ORACLE_TOL,
                     what="rising scores, int8 decode hd 256 vs oracle")


@pytest.mark.parametrize("hd", [64, 128, 256])
def test_prefill_rising_scores_f16(gpu, hd):
    n, n_heads, n_kv = 1000, 4, 2
    say("rescale prefill f16", hd)
    q, k, v = ramp_inputs(7200 + hd, n, n, n_heads, n_kv, hd)
    out = gi_attn.prefill(torch.from_numpy(q).to(gpu), f16_dev(k, gpu), f16_dev(v, gpu), 0, n_heads, n_kv, hd=hd,
                          out_dtype=torch.float32)
    torch.cuda.synchronize()
    want = O.prefill_tc_semantics(q, k, v, 0, n_heads, n_kv, hd=hd)
    assert_close(out.cpu().numpy(), want, what=f"rising scores, prefill hd {hd} vs oracle")


@pytest.mark.parametrize("hd", [64, 128, 256])
def test_prefill_rising_scores_i8(gpu, hd):
    n, n_heads, n_kv = 1000, 4, 2
    say("rescale prefill i8", hd)
    q, kc, vc, ks, vs = ramp_inputs(7300 + hd, n, n, n_heads, n_kv, hd, i8=True)
    t = [torch.from_numpy(x).to(gpu) for x in (q, kc, vc, ks, vs)]
    out = gi_attn.prefill(t[0], t[1], t[2], 0, n_heads, n_kv, hd=hd, out_dtype=torch.float32, k_scale=t[3],
                          v_scale=t[4])
    torch.cuda.synchronize()
    want = O.prefill_tc_semantics_i8(q, kc, vc, ks, vs, 0, n_heads, n_kv, hd=hd)
    assert_close(out.cpu().numpy(), want, what=f"rising scores, int8 prefill hd {hd} vs oracle")


@pytest.mark.parametrize("hd", [96, 128])
def test_prefill_rising_scores_f32(gpu, hd):
    # the f32 prompt kernels: exact online softmax in f32, within the split path's bar of float64
    n, n_heads, n_kv = 600, 4, 2
    say("rescale prefill f32", hd)
    q, k, v = ramp_inputs(7400 + hd, n, n, n_heads, n_kv, hd)
    out = gi_attn.prefill(torch.from_numpy(q).to(gpu), f16_dev(k, gpu), f16_dev(v, gpu), 0, n_heads, n_kv, hd=hd,
                          out_dtype=torch.float32, f32=True)
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), reference_f64(q, k, v, 0, n_heads, n_kv, hd=hd), *SPLIT_F64_TOL,
                 what=f"rising scores, f32 prefill hd {hd}")
