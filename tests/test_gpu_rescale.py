"""Scores that keep rising along the sequence, so that every kernel's running maximum moves many times: the decode
kernels' lazy rescale (a wave keeps its reference maximum until a score passes it by 2^8 in p, then scales its O) and
the prefill's (PF_RESCALE_LOG2), and the f32 kernels' exact online softmax. The queries and keys share a direction
whose key component ramps up with the position. For the decode the ramp is a sawtooth: 20 log2 units over a period of
twice a wave's tile stride (4 tiles: 256 keys for 32-key tiles, 512 for the int8 cache's 64, 128 for head size 256's
16), at 16384 keys over 32 query / 8 kv heads, so that every kernel variant's slices hold at least two tiles per wave
and each wave's later tiles pass its first by more than 2^8: the rescale then scales a nonzero O (the slices' maxima
also differ in the merge). For the prefill 30 log2 units over 1000 keys (a row's reference maximum moves every ~270
keys). Bars: the split decode within 2e-5 of float64 (head size 256 over the int8 and 4-bit caches:
attention_decode_tc256's roundings, against the oracle and at the parity bar); the prefill, whose Q and P are rounded
to f16 as the reference's attention_prefill_tc does, against the oracle's restatement of those roundings at the parity
bar (an f16-rounded Q moves scores of this size by more than the float64 bar allows)."""
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


def ramp_inputs(seed, n_tok, ctx, n_heads, n_kv, hd, i8=False, log2_span=30.0, period=None):
    """q [n_tok, n_heads*hd] f32; K/V rows [ctx, n_kv*hd] (f16 bits, or int8 codes with f32 scales [ctx, n_kv] as
    kv_store quantises them): N(0,1) plus, along e = ones/sqrt(hd) in every head, A for the queries and a ramp
    0..B over the positions for the keys (restarting every `period` keys when given), with A*B/sqrt(hd)*log2(e) =
    log2_span."""
    rng = np.random.default_rng(seed)
    e = np.ones(hd, dtype=np.float64) / np.sqrt(hd)
    ab = log2_span * np.sqrt(hd) / np.log2(np.e)
    A = np.sqrt(ab / 2.0)
    B = ab / A
    q = rng.standard_normal((n_tok, n_heads, hd)) + A * e
    phase = np.arange(ctx) / max(ctx - 1, 1) if period is None else (np.arange(ctx) % period) / (period - 1)
    k = rng.standard_normal((ctx, n_kv, hd)) + (B * phase)[:, None, None] * e
    v = rng.standard_normal((ctx, n_kv, hd))
    q = q.reshape(n_tok, -1).astype(np.float32)
    if i8:
        kc, ks = O.kv_quant_i8(k.astype(np.float32))
        vc, vs = O.kv_quant_i8(v.astype(np.float32))
        return q, kc.reshape(ctx, -1), vc.reshape(ctx, -1), ks, vs
    return q, k.reshape(ctx, -1).astype(np.float16).view(np.uint16), v.reshape(ctx, -1).astype(np.float16).view(np.uint16)


def f16_dev(x, dev):
    return torch.from_numpy(np.ascontiguousarray(x).view(np.int16)).to(dev).view(torch.float16)


DEC_CTX = 16384


def dec_period(hd, i8, n_tok, n_heads, n_kv):
    """The sawtooth's period for a decode case: twice the stride between a wave's tiles when the 4 waves of a
    workgroup take a slice's tiles in turn (tiles of 32 keys, the int8 cache's 64 at head sizes 64 and 128, 16 at
    256); checks that the case's slices hold at least two tiles per wave (at head size 256 two pair sets of two
    waves each can split the slice, so their waves' tiles are half as far apart and see the same rise twice as
    often)."""
    tile = 16 if hd == 256 else 64 if i8 else 32
    if hd in (64, 128, 256):
        chunk = gi_attn.decode_plan(DEC_CTX, n_tok, n_heads, n_kv, hd=hd)[0]
        if i8 and hd != 256:
            chunk = max(chunk, 8 * tile)  # the int8 slice unit (4 tiles of 64 keys); the plan above is f16's
        assert chunk >= 2 * 4 * tile, (hd, i8, n_tok, chunk)
    return 2 * 4 * tile


@pytest.mark.parametrize("hd", [64, 128, 256, 80])
@pytest.mark.parametrize("n_tok", [1, 8])
def test_decode_rising_scores_f16(gpu, hd, n_tok):
    ctx, n_heads, n_kv = DEC_CTX, 32, 8
    say("rescale decode f16", hd, n_tok)
    q, k, v = ramp_inputs(7000 + hd + n_tok, n_tok, ctx, n_heads, n_kv, hd, log2_span=20.0,
                          period=dec_period(hd, False, n_tok, n_heads, n_kv))
    pos0 = ctx - n_tok
    out = gi_attn.decode(torch.from_numpy(q).to(gpu), f16_dev(k, gpu), f16_dev(v, gpu), pos0, n_heads, n_kv, hd=hd)
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), reference_f64(q, k, v, pos0, n_heads, n_kv, hd=hd), *SPLIT_F64_TOL,
                 what=f"rising scores, decode hd {hd}")


@pytest.mark.parametrize("hd", [64, 128, 256])
@pytest.mark.parametrize("n_tok", [1, 8])
def test_decode_rising_scores_i8(gpu, hd, n_tok):
    ctx, n_heads, n_kv = DEC_CTX, 32, 8
    say("rescale decode i8", hd, n_tok)
    q, kc, vc, ks, vs = ramp_inputs(7100 + hd + n_tok, n_tok, ctx, n_heads, n_kv, hd, i8=True, log2_span=20.0,
                                    period=dec_period(hd, True, n_tok, n_heads, n_kv))
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


def ramp_inputs_q4(seed, n_tok, ctx, n_heads, n_kv, log2_rise=23.0, period=128):
    """4-bit cache inputs (head size 256, the reference layout) whose scores rise within every `period` keys and fall
    back at each period's start: key nibbles 9..15 (values +1..+7), key scales in a sawtooth over the positions, and
    queries with a positive component along ones/16, so that a key's score grows with its scale, by about log2_rise
    log2 units over a period. A split-K wave reads 16-key tiles 64 keys apart, so in every slice of at least 128
    keys its second tile's scores pass its first's by more than the 2^8 of the lazy rescale, which then scales a
    nonzero O. Values as make_inputs_q4's (random nibbles 1..15, scales in [0.2, 0.35])."""
    rng = np.random.default_rng(seed)
    A = 4.0
    q = (rng.standard_normal((n_tok, n_heads, 256)) + A / 16.0).reshape(n_tok, -1).astype(np.float32)

    def pack(n):
        return (n[:, 0::2] | (n[:, 1::2] << 4)).astype(np.uint8)

    kn = rng.integers(9, 16, (ctx, n_kv * 256), dtype=np.uint8)
    vn = rng.integers(1, 16, (ctx, n_kv * 256), dtype=np.uint8)
    # score ~ scale * mean(n - 8) * 256 * (A / 16) / 16 * log2(e) = scale * 4 * A * log2(e)
    amp = log2_rise / (4.0 * A * np.log2(np.e))
    ksr = 0.05 + amp * (np.arange(ctx) % period) / (period - 1)
    ks = np.repeat(ksr[:, None], n_kv * 8, axis=1).astype(np.float16).view(np.uint16)
    vs = rng.uniform(0.2, 0.35, (ctx, n_kv * 8)).astype(np.float16).view(np.uint16)
    return q, pack(kn), pack(vn), ks, vs


@pytest.mark.parametrize("n_tok", [1, 8])
def test_decode_rising_scores_q4(gpu, n_tok):
    # the 4-bit kernels (one column block up to 16 pairs per kv head, two per wave above) with their running
    # maximum moving many times in every slice, against the oracle's tc256 roundings and float64
    from attn_common import reference_f64_q4
    from test_gpu_q4 import F64_TOL, q4_dev
    ctx, n_heads, n_kv = 16384, 16, 2
    say("rescale decode q4", n_tok)
    assert gi_attn.decode_plan(ctx, n_tok, n_heads, n_kv, hd=256)[0] >= 128  # at least two tiles per wave
    q, kc, vc, ks, vs = ramp_inputs_q4(7200 + n_tok, n_tok, ctx, n_heads, n_kv)
    pos0 = ctx - n_tok
    out = gi_attn.decode_q4(*q4_dev(q, kc, vc, ks, vs, gpu, n_kv), pos0, n_heads, n_kv)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert_close(got, O.decode_tc256_q4(q, kc, vc, ks, vs, pos0, n_heads, n_kv), *REF_ORACLE_TOL,
                 what="rising scores, q4 decode vs oracle")
    assert_close(got, reference_f64_q4(q, kc, vc, ks, vs, pos0, n_heads, n_kv), *F64_TOL,
                 what="rising scores, q4 decode vs f64")
