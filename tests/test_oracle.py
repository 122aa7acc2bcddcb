"""Pins the CPU oracle (oracle/gi_oracle.cpp) before it is trusted as the GPU path's checker.

The reference has no attention test and no golden vector for this path (its tests cover the f16
conversion only, src/quant.rs:1160-1169). So each oracle function is pinned here by checks a plausible
mistake (a dropped term, a wrong index, a missing scale, a wrong causal bound) would fail:
  - the reference's own known values for the f16 conversion, and an exhaustive check against numpy;
  - an independent float64 softmax attention (tests/attn_common.py) on small shapes;
  - closed forms: one visible position -> V0; zero keys -> the mean of V; one dominant key -> its V row;
  - invariants: the split count (thread count) does not change the result; causality; GQA symmetry;
  - torch's scaled_dot_product_attention as a library cross-check;
  - the committed golden fixtures (tests/golden/), made by tests/golden/make_golden.py in float64.
"""
import math
import os

import numpy as np
import pytest
import torch

import gi_oracle as O
from attn_common import (assert_close, errors, make_inputs, make_inputs_i8, make_inputs_q4, reference_f64, reference_f64_i8,
                         reference_f64_q4)

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


# ---------------------------------------------------------------- f16 conversion (src/quant.rs:10-60)

def test_f16_known_values_from_reference_test():
    # src/quant.rs:1160-1169: round trips within 1e-3 relative, exact 0x3c00 -> 1.0 and 0xc000 -> -2.0
    for v in [0.0, 1.0, -2.5, 0.000061035156, 65504.0, 3.1415927, 1e-7]:
        back = O.f16_bits_to_f32(O.f32_to_f16_bits(np.array([v], np.float32)))[0]
        assert abs(back - v) <= abs(v) * 1e-3 + 1e-7, (v, back)
    assert O.lib().gio_f16_to_f32(0x3C00) == 1.0
    assert O.lib().gio_f16_to_f32(0xC000) == -2.0


def test_f16_to_f32_exhaustive():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = O.f16_bits_to_f32(bits)
    want = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f32_to_f16_round_to_nearest_even():
    rng = np.random.default_rng(7)
    x = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, 200000),
        # halfway cases between adjacent f16 values (ties to even), subnormals, overflow, specials
        (np.arange(-2048, 2048, dtype=np.float32) + 0.5) * np.float32(2.0 ** -10),
        np.float32(2.0 ** -24) * np.arange(0, 64, dtype=np.float32) / 4,
        np.array([65504, 65519.99, 65520, 1e30, -1e30, np.inf, -np.inf, 0.0, -0.0], np.float32),
    ]).astype(np.float32)
    got = O.f32_to_f16_bits(x)
    want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)
    nanbits = O.f32_to_f16_bits(np.array([np.nan], np.float32))[0]
    assert (nanbits & 0x7C00) == 0x7C00 and (nanbits & 0x3FF) != 0


def test_dot_f32_lanes():
    # 8 partial sums then the tail (src/quant.rs:758-768): equal to the exact sum for integer inputs,
    # and to a float64 dot within f32 rounding for random ones
    a = np.arange(1, 20, dtype=np.float32)
    b = np.arange(20, 1, -1, dtype=np.float32)[:19]
    assert O.dot_f32(a, b) == float(np.dot(a.astype(np.float64), b))
    rng = np.random.default_rng(3)
    x, y = rng.standard_normal(131).astype(np.float32), rng.standard_normal(131).astype(np.float32)
    assert abs(O.dot_f32(x, y) - float(np.dot(x.astype(np.float64), y))) < 1e-4
    # the lane structure: 8 lanes summed in order, then + tail
    acc = np.zeros(8, np.float32)
    for c in range(0, 128, 8):
        acc += x[c:c + 8] * y[c:c + 8]
    tail = np.float32(0)
    for i in range(128, 131):
        tail = np.float32(tail + x[i] * y[i])
    s = np.float32(0)
    for v in acc:
        s = np.float32(s + v)
    assert O.dot_f32(x, y) == float(np.float32(s + tail))


# ---------------------------------------------------------------- slice arithmetic (src/cuda.rs:1642, 8426-8444)

def test_slice_arithmetic_at_configs():
    # worked values for the configs: want = ceil(96 / n_kv); chunk = clamp(ceil(span / want), 32, 128)
    assert O.att_want(8) == 12 and O.att_want(4) == 24
    assert O.att_chunk(4096, 12) == 128 and -(-4096 // 128) == 32        # C1: nsplit 32
    assert O.att_chunk(65536, 24) == 128 and -(-65536 // 128) == 512     # C2: nsplit 512
    assert O.att_chunk(32, 24) == 256 and O.att_chunk(33, 24) == 32     # one block up to 32 positions
    assert O.att_chunk(1000, 24) == 42
    # max_splits over spans 1..ctx equals the brute-force maximum
    for ctx in (1, 31, 32, 33, 100, 777, 4096):
        want = O.att_want(4)
        brute = max(-(-s // O.att_chunk(s, want)) for s in range(1, ctx + 1))
        assert O.max_splits(ctx, want) == brute


# ---------------------------------------------------------------- Model::attention (src/model.rs:1320-1409)

SHAPES = [
    # (n_tok, pos0, n_heads, n_kv)
    (1, 0, 4, 1),
    (1, 1, 8, 2),
    (1, 30, 8, 1),
    (1, 31, 32, 8),
    (1, 32, 32, 4),
    (1, 127, 8, 8),
    (1, 128, 32, 4),
    (3, 60, 16, 2),
    (8, 200, 32, 4),
    (20, 5, 8, 1),
]


@pytest.mark.parametrize("n_tok,pos0,n_heads,n_kv", SHAPES)
@pytest.mark.parametrize("threads", [1, 3, 8])
def test_attention_matches_f64(n_tok, pos0, n_heads, n_kv, threads):
    q, k, v = make_inputs(11 + pos0, n_tok, pos0 + n_tok, n_heads, n_kv)
    got = O.attention(q, k, v, pos0, n_heads, n_kv, threads=threads)
    want = reference_f64(q, k, v, pos0, n_heads, n_kv)
    assert_close(got, want, max_abs=2e-5, rel_l2=2e-6, what="oracle vs f64")


def test_attention_f32_cache_equals_widened_f16_cache():
    q, k, v = make_inputs(5, 2, 300, 8, 2)
    a = O.attention(q, k, v, 298, 8, 2)
    b = O.attention(q, O.f16_bits_to_f32(k), O.f16_bits_to_f32(v), 298, 8, 2)
    assert np.array_equal(a, b)


def test_attention_split_invariance_long():
    # splits = min(ceil(threads / pairs), ceil(span / 64)): 1, 4 and 16 slices must agree closely
    q, k, v = make_inputs(21, 1, 4096, 8, 4)
    outs = [O.attention(q, k, v, 4095, 8, 4, threads=t) for t in (1, 16, 64)]
    for o in outs[1:]:
        assert errors(o, outs[0])[0] < 1e-6


def test_closed_form_single_position_is_v0():
    q, k, v = make_inputs(3, 1, 1, 8, 2)
    out = O.attention(q, k, v, 0, 8, 2).reshape(8, 128)
    vv = O.f16_bits_to_f32(v).reshape(2, 128)
    for h in range(8):
        assert np.array_equal(out[h], vv[h // 4])


def test_closed_form_zero_keys_give_mean_of_v():
    q, k, v = make_inputs(4, 1, 777, 8, 2)
    k[:] = 0
    out = O.attention(q, k, v, 776, 8, 2).reshape(8, 128)
    mean = O.f16_bits_to_f32(v).astype(np.float64).reshape(777, 2, 128).mean(axis=0)
    for h in range(8):
        assert np.abs(out[h] - mean[h // 4]).max() < 1e-5


def test_closed_form_dominant_key_selects_its_v_row():
    q, k, v = make_inputs(6, 1, 500, 4, 1)
    q[:] = 0
    q[0, :128] = 1.0  # head 0 only
    kk = k.view(np.float16)
    kk[:] = 0
    kk[321, :] = np.float16(8.0)  # score 8*128/sqrt(128) ~ 90.5 above the rest
    out = O.attention(q, k, v, 499, 4, 1).reshape(4, 128)
    vv = O.f16_bits_to_f32(v)
    assert np.abs(out[0] - vv[321]).max() < 1e-6


def test_causality():
    q, k, v = make_inputs(8, 5, 100, 8, 2)
    a = O.attention(q, k, v, 95, 8, 2)
    k2, v2 = k.copy(), v.copy()
    k2[98:] = 0x3C00
    v2[98:] = 0x4000
    b = O.attention(q, k2, v2, 95, 8, 2)
    # tokens at positions 95..97 see keys 0..97 only; tokens 98, 99 see the change
    assert np.array_equal(a[:3], b[:3])
    assert not np.array_equal(a[3:], b[3:])


def test_gqa_heads_with_equal_queries_agree():
    q, k, v = make_inputs(9, 1, 333, 8, 2)
    qq = q.reshape(8, 128)
    qq[1] = qq[0]
    qq[5] = qq[4]
    out = O.attention(q, k, v, 332, 8, 2).reshape(8, 128)
    assert np.array_equal(out[0], out[1]) and np.array_equal(out[4], out[5])
    assert not np.array_equal(out[0], out[4])


def test_matches_torch_sdpa():
    n_heads, n_kv, n, pos0 = 8, 2, 40, 24
    q, k, v = make_inputs(31, n, pos0 + n, n_heads, n_kv)
    got = O.attention(q, k, v, pos0, n_heads, n_kv)
    K = torch.from_numpy(O.f16_bits_to_f32(k)).view(-1, n_kv, 128).double()
    V = torch.from_numpy(O.f16_bits_to_f32(v)).view(-1, n_kv, 128).double()
    Q = torch.from_numpy(q).view(n, n_heads, 128).double()
    G = n_heads // n_kv
    Kx = K.repeat_interleave(G, dim=1).transpose(0, 1)  # [h, t, d]
    Vx = V.repeat_interleave(G, dim=1).transpose(0, 1)
    mask = torch.arange(pos0 + n)[None, :] <= (pos0 + torch.arange(n))[:, None]
    ref = torch.nn.functional.scaled_dot_product_attention(Q.transpose(0, 1), Kx, Vx, attn_mask=mask)
    ref = ref.transpose(0, 1).reshape(n, -1).numpy()
    assert_close(got, ref, max_abs=2e-5, rel_l2=2e-6, what="oracle vs sdpa")


# ---------------------------------------------------------------- GPU-kernel semantics restatements

@pytest.mark.parametrize("n_tok,pos0,n_heads,n_kv", [(1, 0, 32, 8), (1, 31, 32, 8), (1, 32, 32, 4),
                                                     (1, 1000, 32, 4), (8, 4000, 32, 4), (3, 129, 16, 8)])
def test_decode_gpu_semantics_matches_f64(n_tok, pos0, n_heads, n_kv):
    q, k, v = make_inputs(41 + pos0, n_tok, pos0 + n_tok, n_heads, n_kv)
    got = O.decode_gpu_semantics(q, k, v, pos0, n_heads, n_kv)
    want = reference_f64(q, k, v, pos0, n_heads, n_kv)
    assert_close(got, want, max_abs=2e-5, rel_l2=2e-6, what="decode semantics vs f64")


def test_decode_gpu_semantics_butterfly_score_is_a_dot():
    # one position: out = V0 whatever the score; two positions with equal keys: the mean of both values
    q, k, v = make_inputs(2, 1, 2, 8, 1)
    k[1] = k[0]
    out = O.decode_gpu_semantics(q, k, v, 1, 8, 1).reshape(8, 128)
    vv = O.f16_bits_to_f32(v).astype(np.float64)
    assert np.abs(out - (vv[0] + vv[1]) / 2).max() < 1e-6


@pytest.mark.parametrize("n,pos0,n_heads,n_kv", [(64, 0, 8, 2), (100, 0, 4, 1), (70, 130, 8, 4)])
def test_prefill_tc_semantics_within_parity_bar(n, pos0, n_heads, n_kv):
    # the reference's tensor-core prefill rounds Q*scale*log2e and P to f16: within the north star's bar of
    # the exact result, but not equal to it
    q, k, v = make_inputs(51 + n, n, pos0 + n, n_heads, n_kv)
    got = O.prefill_tc_semantics(q, k, v, pos0, n_heads, n_kv)
    want = reference_f64(q, k, v, pos0, n_heads, n_kv)
    ma, rl = assert_close(got, want, what="prefill_tc semantics vs f64")
    assert ma > 1e-6  # the f16 roundings are visible


def _f16(x):
    return np.float32(np.float16(np.float32(x)))


def _q_between_f16(hd, n_heads, x):
    """A query row whose every element, times scale*log2(e) in f32, is x (not an f16 value)."""
    qs = np.float32(1.0 / math.sqrt(hd)) * np.float32(1.4426950408889634)
    q = np.full((1, n_heads * hd), np.float32(np.float64(x) / np.float64(qs)), dtype=np.float32)
    assert q[0, 0] * qs != _f16(q[0, 0] * qs)  # the product is not an f16 value: its rounding matters
    return q, qs


@pytest.mark.parametrize("hd", [64, 128])
def test_prefill_tc_semantics_roundings_by_hand(hd):
    # One query at position 1 over two keys: key 0 all ones, key 1 zero; value 0 all ones, value 1 zero. Each
    # element of Q*scale*log2e is 2^-7 (1 + 1.25 * 2^-10) (head size 64: 2^-6 (...)), which f16 rounds down to
    # 2^-7 (1 + 2^-10), so the score of key 0 is 128 * that = 1 + 2^-10 exactly (unrounded: 1 + 1.25 * 2^-10).
    # Then P0 = 1, P1 = f16(exp2(-(1 + 2^-10))), l = P0 + P1 (the rounded P), out = P0 / l in every dim.
    x = (128.0 / hd) * 2.0 ** -7 * (1 + 1.25 * 2.0 ** -10)
    q, qs = _q_between_f16(hd, 1, x)
    k = np.zeros((2, hd), np.float16)
    k[0] = 1
    v = np.zeros((2, hd), np.float16)
    v[0] = 1
    got = O.prefill_tc_semantics(q, k.view(np.uint16), v.view(np.uint16), 1, 1, 1, hd=hd)
    s0 = np.float32(hd) * _f16(q[0, 0] * qs)
    assert s0 == np.float32(1 + 2.0 ** -10)
    p1 = _f16(np.exp2(-s0))
    want = np.float32(1) / (np.float32(1) + p1)
    np.testing.assert_allclose(got, want, rtol=2e-7, atol=0)
    # each plausible slip moves the result far beyond that tolerance
    s0_unrounded = np.float32(hd) * (q[0, 0] * qs)
    slips = {"Q not rounded": 1 / (1 + _f16(np.exp2(-s0_unrounded))),
             "P not rounded": 1 / (1 + np.exp2(-s0)),
             "natural-log softmax": 1 / (1 + _f16(np.exp(-s0)))}
    for what, alt in slips.items():
        assert abs(float(alt) - float(want)) > 1e-5, what


def test_decode_tc256_i8_roundings_by_hand():
    # attention_decode_tc256 over the int8 cache, one token at position 1 over two keys (one 8-position tile):
    # key 0 all ones (scale 1), key 1 zero; each element of Q*scale*log2e is 2^-8 (1 + 1.25 * 2^-10), which
    # f16 rounds down, so score 0 = 256 * 2^-8 (1 + 2^-10) = 1 + 2^-10 exactly and score 1 = 0. Values: row 0
    # all 1 with scale 1/3, row 1 all 2 with scale 1/5. P = f16(p * vscale * 2^10): P0 = f16(1024/3) = 341.25,
    # P1 = f16(2^-(1 + 2^-10) * 1024/5); l = 1 + 2^-(1 + 2^-10) (the unrounded p); out = (P0 + 2 P1) / 1024 / l.
    x = 2.0 ** -8 * (1 + 1.25 * 2.0 ** -10)
    q, qs = _q_between_f16(256, 1, x)
    k = np.zeros((2, 256), np.int8)
    k[0] = 1
    v = np.zeros((2, 256), np.int8)
    v[0], v[1] = 1, 2
    ks = np.ones((2, 1), np.float32)
    vs = np.array([[1 / 3], [1 / 5]], np.float32)
    got = O.decode_tc256_i8(q, k, v, ks, vs, 1, 1, 1)
    s0 = np.float32(256) * _f16(q[0, 0] * qs)
    assert s0 == np.float32(1 + 2.0 ** -10)
    p1 = np.exp2(-s0)
    P0 = _f16(np.float32(1) * (vs[0, 0] * np.float32(1024)))
    P1 = _f16(p1 * (vs[1, 0] * np.float32(1024)))
    assert P0 == np.float32(341.25)
    want = (P0 + np.float32(2) * P1) * (np.float32(1) / np.float32(1024) / (np.float32(1) + p1))
    np.testing.assert_allclose(got, want, rtol=2e-7, atol=0)
    s0_unrounded = np.float32(256) * (q[0, 0] * qs)
    p1u = np.exp2(-s0_unrounded)
    slips = {"Q not rounded": (P0 + 2 * _f16(p1u * vs[1, 0] * 1024)) / 1024 / (1 + p1u),
             "l of the rounded P": (P0 + 2 * P1) / (P0 + P1),
             "P not rounded": (vs[0, 0] * 1024 + 2 * p1 * vs[1, 0] * 1024) / 1024 / (1 + p1),
             "value scale in l": (P0 + 2 * P1) / 1024 / (vs[0, 0] + p1 * vs[1, 0]) / 1024}
    for what, alt in slips.items():
        assert abs(float(alt) - float(want)) > 1e-5 * float(want), what


@pytest.mark.parametrize("hd", [64, 128, 256])
def test_prefill_tc_i8_roundings_by_hand(hd):
    # attn_prefill_tc over the int8 cache (src/cuda.rs:2466-2498, 2548-2605), one query at position 1 over two
    # keys: key 0 all ones (scale 1), key 1 zero; Q*scale*log2e rounds to f16 so that score 0 = 1 + 2^-10
    # exactly. Values: row 0 all 1 with scale 1/3, row 1 all 2 with scale 1/5 (non-unit, so every rounding step
    # shows). The reference biases each value scale by 2^10 as it loads it, rounds p * (vscale * 2^10) to f16
    # for P V, sums the f16-rounded p into l, and scales the output by (2^-10 / l).
    x = (128.0 / hd) * 2.0 ** -7 * (1 + 1.25 * 2.0 ** -10)
    q, qs = _q_between_f16(hd, 1, x)
    k = np.zeros((2, hd), np.int8)
    k[0] = 1
    v = np.zeros((2, hd), np.int8)
    v[0], v[1] = 1, 2
    ks = np.ones((2, 1), np.float32)
    vs = np.array([[1 / 3], [1 / 5]], np.float32)
    got = O.prefill_tc_semantics_i8(q, k, v, ks, vs, 1, 1, 1, hd=hd)
    s0 = np.float32(hd) * _f16(q[0, 0] * qs)
    assert s0 == np.float32(1 + 2.0 ** -10)
    p1 = np.exp2(np.float32(0) - s0)
    b0, b1 = vs[0, 0] * np.float32(1024), vs[1, 0] * np.float32(1024)
    P0, P1 = _f16(np.float32(1) * b0), _f16(p1 * b1)
    assert P0 == np.float32(341.25)
    lsum = np.float32(1) + _f16(p1)
    want = (P0 + np.float32(2) * P1) * ((np.float32(1) / np.float32(1024)) / lsum)
    np.testing.assert_allclose(got, want, rtol=2e-7, atol=0)
    slips = {"round p, then times the value scale": (P0 + 2 * _f16(_f16(p1) * b1)) / 1024 / lsum,
             "l of p times the value scale": (P0 + 2 * P1) / (P0 + P1),
             "P V of the unrounded product": (b0 + 2 * p1 * b1) / 1024 / lsum,
             "l of the unrounded p": (P0 + 2 * P1) / 1024 / (1 + p1)}
    for what, alt in slips.items():
        assert abs(float(alt) - float(want)) > 1e-5 * float(want), what


def _q4_two_keys():
    """One rotated query at position 1 over two 4-bit keys (head size 256): key 0 all +1 (nibble 9, scale 1), key
    1 all 0 (nibble 8), so score 0 = 256 * f16(Q*scale*log2e) = 1 + 2^-10 exactly. Values: row 0 all nibble 11
    (+3) with scale f16(1/3), row 1 all nibble 15 (+7) with scale f16(0.3); each value is f16((n - 8) * scale)
    (kv4_pair, src/cuda.rs:238-240), and 7 * f16(0.3) is not an f16 value, so its rounding shows."""
    x = 2.0 ** -8 * (1 + 1.25 * 2.0 ** -10)
    q, qs = _q_between_f16(256, 1, x)
    kc = np.array([[0x99] * 128, [0x88] * 128], np.uint8)
    vc = np.array([[0xBB] * 128, [0xFF] * 128], np.uint8)

    def h(a):
        return np.float16(a).view(np.uint16)

    ks = np.array([[h(1.0)] * 8] * 2, np.uint16)
    vs = np.array([[h(1 / 3)] * 8, [h(0.3)] * 8], np.uint16)
    s0 = np.float32(256) * _f16(q[0, 0] * qs)
    assert s0 == np.float32(1 + 2.0 ** -10)
    vau = np.float32(3) * np.float32(np.float16(1 / 3))
    vbu = np.float32(7) * np.float32(np.float16(0.3))
    va, vb = _f16(vau), _f16(vbu)
    assert vb != vbu
    p1 = np.exp2(np.float32(0) - s0)
    p1u = np.exp2(np.float32(0) - np.float32(256) * (q[0, 0] * qs))  # had Q not been rounded
    return (q, kc, vc, ks, vs), p1, p1u, va, vb, vau, vbu


def test_decode_tc256_q4_roundings_by_hand():
    # attention_decode_tc256 over the 4-bit cache (src/cuda.rs:2681-2760): KV_SCALE is 1, so P = f16(p * 2^10),
    # l sums the unrounded p, and the output is (P V) * (2^-10 / l)
    args, p1, p1u, va, vb, vau, vbu = _q4_two_keys()
    got = O.decode_tc256_q4(*args, 1, 1, 1)
    P0, P1 = _f16(1024), _f16(p1 * np.float32(1024))
    lsum = np.float32(1) + p1
    want = (P0 * va + P1 * vb) * ((np.float32(1) / np.float32(1024)) / lsum)
    np.testing.assert_allclose(got, want, rtol=2e-7, atol=0)
    slips = {"P not rounded": (P0 * va + p1 * 1024 * vb) / 1024 / lsum,
             "l of the rounded P": (P0 * va + P1 * vb) / (P0 + P1),
             "values not rounded": (P0 * vau + P1 * vbu) / 1024 / lsum,
             "Q not rounded": (P0 * va + _f16(p1u * 1024) * vb) / 1024 / (1 + p1u)}
    for what, alt in slips.items():
        assert abs(float(alt) - float(want)) > 1e-5 * float(want), what


def test_prefill_tc256_q4_roundings_by_hand():
    # attn_prefill_tc<256, 2> over the 4-bit cache (src/cuda.rs:2495-2514): the f16 cache's arithmetic over the
    # staged f16 values, so P = f16(p) for both P V and l, and the output is P V / l
    args, p1, p1u, va, vb, vau, vbu = _q4_two_keys()
    got = O.prefill_tc256_q4(*args, 1, 1, 1)
    P1 = _f16(p1)
    lsum = np.float32(1) + P1
    want = (va + P1 * vb) / lsum
    np.testing.assert_allclose(got, want, rtol=2e-7, atol=0)
    slips = {"P not rounded": (va + p1 * vb) / (1 + p1),
             "l of the unrounded p": (va + P1 * vb) / (1 + p1),
             "values not rounded": (vau + P1 * vbu) / lsum,
             "Q not rounded": (va + _f16(p1u) * vb) / (1 + _f16(p1u))}
    for what, alt in slips.items():
        assert abs(float(alt) - float(want)) > 1e-5 * float(want), what


@pytest.mark.parametrize("n_tok,pos0,n_heads,n_kv", [(1, 0, 16, 2), (1, 7, 16, 2), (1, 8, 8, 1), (1, 300, 16, 2),
                                                     (3, 100, 8, 1), (8, 2000, 16, 2), (1, 4095, 16, 16)])
def test_decode_tc256_i8_within_parity_bar(n_tok, pos0, n_heads, n_kv):
    # f16 Q and f16 P*vscale*2^10: within the bar of float64 attention over the dequantised cache, not equal
    q, k, v, ks, vs = make_inputs_i8(91 + pos0, n_tok, pos0 + n_tok, n_heads, n_kv, hd=256)
    got = O.decode_tc256_i8(q, k, v, ks, vs, pos0, n_heads, n_kv)
    want = reference_f64_i8(q, k, v, ks, vs, pos0, n_heads, n_kv, hd=256)
    ma, _ = assert_close(got, want, what="decode_tc256 int8 semantics vs f64")
    assert ma > 1e-6


def test_decode_tc256_i8_slice_count_and_gqa():
    # the result does not depend on the slice count beyond the f16 rounding of P (taken against each warp's
    # running max, which the slicing moves), and heads of one group with equal queries give equal outputs
    q, k, v, ks, vs = make_inputs_i8(17, 2, 3000, 8, 2, hd=256)
    a = O.decode_tc256_i8(q, k, v, ks, vs, 2998, 8, 2)
    b = O.decode_tc256_i8(q, k, v, ks, vs, 2998, 8, 2, cap=4096, want=1)  # one slice per token (48 above)
    ma, _ = errors(a, b)
    assert 0 < ma < 1e-4
    q2 = q.reshape(2, 8, 256).copy()
    q2[:, 1] = q2[:, 0]
    o = O.decode_tc256_i8(q2.reshape(2, -1), k, v, ks, vs, 2998, 8, 2).reshape(2, 8, 256)
    np.testing.assert_array_equal(o[:, 0], o[:, 1])


# ---------------------------------------------------------------- golden fixtures

def _golden_files():
    return sorted(f for f in os.listdir(GOLDEN) if f.endswith(".npz"))


def test_golden_fixtures_exist():
    assert len(_golden_files()) >= 4


@pytest.mark.parametrize("name", _golden_files() if os.path.isdir(GOLDEN) else [])
def test_oracle_against_golden(name):
    z = np.load(os.path.join(GOLDEN, name))
    n_heads, n_kv, pos0 = int(z["n_heads"]), int(z["n_kv"]), int(z["pos0"])
    hd = int(z["hd"]) if "hd" in z.files else 128
    q = z["q"].astype(np.float32)
    if "q4" in z.files:  # the 4-bit cache's tensor-core kernels round Q and P to f16: the parity bar
        fn = O.prefill_tc256_q4 if name.startswith("prefill") else O.decode_tc256_q4
        assert_close(fn(q, z["k"], z["v"], z["ks"], z["vs"], pos0, n_heads, n_kv), z["out"], what=name)
    elif "ks" in z.files and name.startswith("prefill") and hd in (64, 128, 256):  # f16 P * vscale * 2^10: the bar
        got = O.prefill_tc_semantics_i8(q, z["k"], z["v"], z["ks"], z["vs"], pos0, n_heads, n_kv, hd=hd)
        assert_close(got, z["out"], what=name)
    elif "ks" in z.files and hd == 256:  # attention_decode_tc256 rounds Q and P*vscale to f16: the parity bar
        got = O.decode_tc256_i8(q, z["k"], z["v"], z["ks"], z["vs"], pos0, n_heads, n_kv)
        assert_close(got, z["out"], what=name)
    elif "ks" in z.files and hd == 128:  # the int8 split path keeps f32 precision
        got = O.decode_gpu_semantics_i8(q, z["k"], z["v"], z["ks"], z["vs"], pos0, n_heads, n_kv)
        assert_close(got, z["out"], max_abs=2e-5, rel_l2=2e-6, what=name)
    elif "ks" in z.files:  # head size 64 and the f32 kernels' sizes: Model::attention over the dequantised cache
        def deq(c, sc):
            return (c.reshape(c.shape[0], n_kv, hd).astype(np.float32) * sc[:, :, None]).reshape(c.shape[0], -1)

        got = O.attention(q, deq(z["k"], z["ks"]), deq(z["v"], z["vs"]), pos0, n_heads, n_kv, hd=hd)
        assert_close(got, z["out"], max_abs=2e-5, rel_l2=2e-6, what=name)
    else:
        got = O.attention(q, z["k"], z["v"], pos0, n_heads, n_kv, hd=hd)
        assert_close(got, z["out"], max_abs=2e-5, rel_l2=2e-6, what=name)


# ---------------------------------------------------------------- qk_norm_rope (KV store)

def _rope_inputs(seed, n, n_heads, n_kv, hd, cap):
    rng = np.random.default_rng(seed)
    qkv = rng.standard_normal((n, (n_heads + 2 * n_kv) * hd), dtype=np.float32)
    kc = np.zeros((cap, n_kv * hd), dtype=np.uint16)
    return qkv, kc, kc.copy()


def test_rope_position_zero_is_identity_and_cache_rounds_like_numpy():
    qkv, kc, vc = _rope_inputs(1, 2, 4, 2, 128, 4)
    out, kc2, vc2 = O.qk_norm_rope(qkv, kc, vc, 0, 4, 2)
    # token 0 sits at position 0: nothing rotates; token 1 at position 1 does
    np.testing.assert_array_equal(out[0], qkv[0])
    assert not np.array_equal(out[1, :4 * 128], qkv[1, :4 * 128])
    kv = out[:, 4 * 128:].reshape(2, 2, 2 * 128)
    np.testing.assert_array_equal(kc2[:2], kv[:, 0].astype(np.float16).view(np.uint16))
    np.testing.assert_array_equal(vc2[:2], kv[:, 1].astype(np.float16).view(np.uint16))
    assert not kc2[2:].any() and not vc2[2:].any()  # other positions untouched


@pytest.mark.parametrize("neox", [True, False])
def test_rope_keeps_pair_lengths(neox):
    hd, rope_dim = 128, 96
    qkv, kc, vc = _rope_inputs(2, 3, 2, 1, hd, 1300)
    out, _, _ = O.qk_norm_rope(qkv, kc, vc, 1234, 2, 1, rope_dim=rope_dim, neox=neox)
    half = rope_dim // 2
    for h in range(3):  # q heads and the k head
        a = qkv[:, h * hd:(h + 1) * hd].astype(np.float64)
        b = out[:, h * hd:(h + 1) * hd].astype(np.float64)
        ia = np.arange(half) if neox else 2 * np.arange(half)
        ib = ia + half if neox else ia + 1
        np.testing.assert_allclose(np.hypot(b[:, ia], b[:, ib]), np.hypot(a[:, ia], a[:, ib]), rtol=2e-6)
        np.testing.assert_array_equal(b[:, rope_dim:], a[:, rope_dim:])  # partial rotary: the rest unchanged


@pytest.mark.parametrize("neox,use_ff", [(True, False), (False, False), (True, True)])
def test_rope_one_hot_lands_on_its_partner(neox, use_ff):
    hd, base, pos = 64, 500000.0, 37
    half = hd // 2
    ff = (1.0 + np.arange(half, dtype=np.float32) / 7).astype(np.float32) if use_ff else None
    for i in (0, 1, 5, half - 1):
        ia = i if neox else 2 * i
        ib = ia + half if neox else ia + 1
        qkv = np.zeros((1, 3 * hd), dtype=np.float32)
        qkv[0, ia] = 1.0
        out, _, _ = O.qk_norm_rope(qkv, np.zeros((64, hd), np.uint16), np.zeros((64, hd), np.uint16), pos, 1, 1, hd=hd,
                                   base=base, ff=ff, neox=neox)
        theta = pos * base ** (-2.0 * i / hd) / (ff[i] if use_ff else 1.0)  # float64
        assert abs(out[0, ia] - math.cos(theta)) < 2e-6
        assert abs(out[0, ib] - math.sin(theta)) < 2e-6
        assert np.count_nonzero(out[0, :hd]) <= 2


def test_rms_norm_gives_unit_rms_times_weights():
    hd = 128
    qkv, kc, vc = _rope_inputs(3, 2, 2, 1, hd, 2)
    w = np.random.default_rng(9).uniform(0.5, 2.0, hd).astype(np.float32)
    out, _, _ = O.qk_norm_rope(qkv, kc, vc, 0, 2, 1, qn=np.ones(hd, np.float32), kn=w)
    # token 0 (position 0, unrotated): q heads have RMS 1, the k head is normalised then weighted
    for h in range(2):
        assert abs(np.sqrt(np.mean(out[0, h * hd:(h + 1) * hd].astype(np.float64) ** 2)) - 1.0) < 1e-6
    k = qkv[0, 2 * hd:3 * hd].astype(np.float64)
    want = k / np.sqrt(np.mean(k ** 2) + 1e-6) * w
    np.testing.assert_allclose(out[0, 2 * hd:3 * hd], want, rtol=1e-5, atol=1e-6)


# ---------------------------------------------------------------- int8 cache (KV8)

def test_kv_quant_i8_closed_forms():
    hd = 128
    x = np.zeros((4, hd), dtype=np.float32)
    # row 0: all zero -> scale 0 and zero bytes (inv = 0, no division by zero)
    # row 1: max |x| = 127 -> scale exactly 1, so integers are kept and halves round to even
    x[1, :8] = [127, -3, 2.5, 3.5, -0.5, -1.5, 0.49, -126.5]
    # row 2: max |x| = 127 * 2^-5 -> scale 2^-5 exactly; multiples of 2^-5 map to their integers
    ints = np.arange(-127, 1, dtype=np.float32)
    x[2, :128] = ints * 2.0 ** -5
    # row 3: negative extreme -> -127
    x[3, 7] = -3.0
    x[3, 9] = 1.0
    q, sc = O.kv_quant_i8(x)
    assert sc[0] == 0 and not q[0].any()
    assert sc[1] == 1.0
    np.testing.assert_array_equal(q[1, :8], [127, -3, 2, 4, 0, -2, 0, -126])
    assert sc[2] == 2.0 ** -5
    np.testing.assert_array_equal(q[2], ints.astype(np.int8))
    assert q[3, 7] == -127 and q[3, 9] == round(127 / 3)


def test_kv_quant_i8_error_bound_and_extremes():
    x = np.random.default_rng(5).standard_normal((64, 256), dtype=np.float32) * np.float32(3)
    q, sc = O.kv_quant_i8(x)
    err = np.abs(q.astype(np.float64) * sc[:, None] - x)
    assert np.all(err <= sc[:, None] * (0.5 + 1e-5))
    np.testing.assert_array_equal(np.abs(q.astype(np.int32)).max(axis=1), 127)  # each row's max maps to +-127
    np.testing.assert_allclose(sc, np.abs(x).max(axis=1) / 127, rtol=1e-6)


@pytest.mark.parametrize("n_tok,pos0,n_heads,n_kv", [(1, 0, 32, 8), (1, 33, 32, 4), (1, 1000, 32, 4),
                                                     (5, 300, 16, 8), (8, 2000, 32, 4)])
def test_decode_gpu_semantics_i8_matches_f64(n_tok, pos0, n_heads, n_kv):
    q, k, v, ks, vs = make_inputs_i8(61 + pos0, n_tok, pos0 + n_tok, n_heads, n_kv)
    got = O.decode_gpu_semantics_i8(q, k, v, ks, vs, pos0, n_heads, n_kv)
    want = reference_f64_i8(q, k, v, ks, vs, pos0, n_heads, n_kv)
    assert_close(got, want, max_abs=2e-5, rel_l2=2e-6, what="int8 decode semantics vs f64")


def test_decode_i8_unit_scales_equal_the_f16_path():
    # small integers are exact in f16 and unit scales multiply exactly: both restatements must agree bit for bit
    q, k, v, _, _ = make_inputs_i8(7, 3, 700, 16, 4)
    k = (k // 8).astype(np.int8)  # keep scores moderate
    ones = np.ones((700, 4), dtype=np.float32)
    got = O.decode_gpu_semantics_i8(q, k, v, ones, ones, 697, 16, 4)
    kb = k.astype(np.float16).view(np.uint16)
    vb = v.astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(got, O.decode_gpu_semantics(q, kb, vb, 697, 16, 4))


@pytest.mark.parametrize("hd,neox", [(128, True), (64, False), (256, True)])
def test_rope_i8_stores_the_quantised_rows(hd, neox):
    n_heads, n_kv, n, pos0, cap = 4, 2, 3, 50, 60
    rng = np.random.default_rng(hd)
    qkv = rng.standard_normal((n, (n_heads + 2 * n_kv) * hd), dtype=np.float32)
    qn = rng.uniform(0.5, 1.5, hd).astype(np.float32)
    kn = rng.uniform(0.5, 1.5, hd).astype(np.float32)
    kc = np.zeros((cap, n_kv * hd), np.int8)
    sc = np.full((cap, n_kv), -1.0, np.float32)
    out, kc8, vc8, ks, vs = O.qk_norm_rope_i8(qkv, kc, kc, sc, sc, pos0, n_heads, n_kv, hd=hd, qn=qn, kn=kn,
                                             neox=neox)
    # the rows themselves are the f16 path's
    out16, _, _ = O.qk_norm_rope(qkv, np.zeros((cap, n_kv * hd), np.uint16), np.zeros((cap, n_kv * hd), np.uint16),
                                 pos0, n_heads, n_kv, hd=hd, qn=qn, kn=kn, neox=neox)
    np.testing.assert_array_equal(out, out16)
    k_rows = out[:, n_heads * hd:(n_heads + n_kv) * hd]
    v_rows = qkv[:, (n_heads + n_kv) * hd:]
    for cache, scales, rows in ((kc8, ks, k_rows), (vc8, vs, v_rows)):
        got = cache[pos0:pos0 + n].reshape(n, n_kv, hd).astype(np.float64) * scales[pos0:pos0 + n, :, None]
        want = rows.reshape(n, n_kv, hd)
        assert np.all(np.abs(got - want) <= scales[pos0:pos0 + n, :, None] * (0.5 + 1e-5))
        np.testing.assert_allclose(scales[pos0:pos0 + n], np.abs(want).max(axis=2) / 127, rtol=1e-6)
        assert not cache[:pos0].any() and not cache[pos0 + n:].any()
        assert np.all(scales[:pos0] == -1) and np.all(scales[pos0 + n:] == -1)


@pytest.mark.parametrize("n,pos0,n_heads,n_kv", [(64, 0, 8, 2), (100, 0, 4, 1), (70, 130, 8, 4)])
def test_prefill_tc_semantics_i8_within_parity_bar(n, pos0, n_heads, n_kv):
    # the reference's int8 prefill rounds Q*scale*log2e, P and P*vscale to f16: within the bar of the exact
    # attention over the dequantised cache
    q, k, v, ks, vs = make_inputs_i8(71 + n, n, pos0 + n, n_heads, n_kv)
    got = O.prefill_tc_semantics_i8(q, k, v, ks, vs, pos0, n_heads, n_kv)
    want = reference_f64_i8(q, k, v, ks, vs, pos0, n_heads, n_kv)
    ma, _ = assert_close(got, want, what="int8 prefill semantics vs f64")
    assert ma > 1e-6  # the f16 roundings are visible


def test_prefill_i8_unit_scales_follow_the_f16_path():
    # unit scales and small integers: the int8 restatement differs from the f16 one only by where P*1024
    # rounds (the 2^10 bias keeps tiny probabilities normal), far below the f16 step of P itself
    q, k, v, _, _ = make_inputs_i8(8, 80, 200, 8, 2)
    k = (k // 16).astype(np.int8)
    ones = np.ones((200, 2), dtype=np.float32)
    got = O.prefill_tc_semantics_i8(q, k, v, ones, ones, 120, 8, 2)
    want = O.prefill_tc_semantics(q, k.astype(np.float16).view(np.uint16), v.astype(np.float16).view(np.uint16), 120,
                                  8, 2)
    np.testing.assert_allclose(got, want, rtol=0, atol=1e-4)


@pytest.mark.parametrize("n,pos0,n_heads,n_kv", [(48, 0, 4, 2), (70, 33, 4, 1)])
def test_prefill_tc_semantics_hd256_within_parity_bar(n, pos0, n_heads, n_kv):
    # attention_prefill_tc256's arithmetic (head size 256): within the bar of the exact attention, and its
    # first 128 dims of V feed the first 128 output dims only (a head of 256 = two halves of P V)
    q, k, v = make_inputs(81 + n, n, pos0 + n, n_heads, n_kv, hd=256)
    got = O.prefill_tc_semantics(q, k, v, pos0, n_heads, n_kv, hd=256)
    want = reference_f64(q, k, v, pos0, n_heads, n_kv, hd=256)
    ma, _ = assert_close(got, want, what="prefill_tc hd256 semantics vs f64")
    assert ma > 1e-6
    v2 = v.reshape(v.shape[0], n_kv, 256).copy()
    v2[:, :, 128:] = 0
    got2 = O.prefill_tc_semantics(q, k, v2.reshape(v.shape), pos0, n_heads, n_kv, hd=256).reshape(n, n_heads, 256)
    np.testing.assert_array_equal(got2[:, :, :128], got.reshape(n, n_heads, 256)[:, :, :128])
    assert not got2[:, :, 128:].any()


@pytest.mark.parametrize("n,pos0,n_heads,n_kv,i8", [(48, 0, 9, 3, False), (70, 33, 4, 1, False), (48, 0, 9, 3, True),
                                                    (70, 33, 4, 1, True)])
def test_prefill_tc_semantics_hd64_within_parity_bar(n, pos0, n_heads, n_kv, i8):
    # attention_prefill_tc64's arithmetic (head size 64, f16 and int8 caches): within the bar of the exact attention,
    # its f16 roundings visible; and the head-64 restatement is the head-128 one on rows zero-padded to 128 dims
    # (padding adds nothing to a dot product or to P V), with the scale passed explicitly
    if i8:
        q, k, v, ks, vs = make_inputs_i8(91 + n, n, pos0 + n, n_heads, n_kv, hd=64)
        got = O.prefill_tc_semantics_i8(q, k, v, ks, vs, pos0, n_heads, n_kv, hd=64)
        want = reference_f64_i8(q, k, v, ks, vs, pos0, n_heads, n_kv, hd=64)
    else:
        q, k, v = make_inputs(91 + n, n, pos0 + n, n_heads, n_kv, hd=64)
        got = O.prefill_tc_semantics(q, k, v, pos0, n_heads, n_kv, hd=64)
        want = reference_f64(q, k, v, pos0, n_heads, n_kv, hd=64)
    ma, _ = assert_close(got, want, what="prefill_tc hd64 semantics vs f64")
    assert ma > 1e-6

    def pad(x, rows, heads):
        y = np.zeros((rows, heads, 128), dtype=x.dtype)
        y[:, :, :64] = x.reshape(rows, heads, 64)
        return y.reshape(rows, heads * 128)

    qp = pad(q, n, n_heads)
    if i8:
        padded = O.prefill_tc_semantics_i8(qp, pad(k, k.shape[0], n_kv), pad(v, v.shape[0], n_kv), ks, vs, pos0,
                                           n_heads, n_kv, scale=1 / 8.0, hd=128)
    else:
        padded = O.prefill_tc_semantics(qp, pad(k, k.shape[0], n_kv), pad(v, v.shape[0], n_kv), pos0, n_heads, n_kv,
                                        scale=1 / 8.0, hd=128)
    np.testing.assert_array_equal(padded.reshape(n, n_heads, 128)[:, :, :64].reshape(n, -1), got)


# ---------------------------------------------------------------- the 4-bit cache (KV4)

def _sylvester(n):
    """H[i][j] = (-1)^popcount(i & j): the unnormalized Sylvester-order Walsh-Hadamard matrix."""
    i = np.arange(n)
    bits = np.vectorize(lambda x: bin(x).count("1"))(i[:, None] & i[None, :])
    return np.where(bits % 2 == 0, 1, -1).astype(np.int64)


def test_kv4_fwht_matches_the_matrix_and_is_its_own_inverse():
    # src/hadamard.rs:201-219's test (x_i = sin(0.37 i), the matrix (-1)^popcount(i&j) / sqrt(n), applied twice
    # gives x back) at the cache's 256 points
    x = np.sin(np.arange(256) * 0.37).astype(np.float32)[None, :]
    y = O.kv4_fwht(x)
    want = (_sylvester(256) @ x[0].astype(np.float64)) / 16.0
    np.testing.assert_allclose(y[0], want, rtol=0, atol=1e-5)
    np.testing.assert_allclose(O.kv4_fwht(y), x, rtol=0, atol=1e-5)


def test_kv4_fwht_exact_on_integers_and_unit_vectors():
    # small integers: every butterfly sum is exact in f32 and so is the 1/16, so the result equals the integer
    # matrix product / 16 bit for bit (any order of the stages would); unit vector e_j gives column j / 16
    rng = np.random.default_rng(5)
    x = rng.integers(-1000, 1000, (6, 256)).astype(np.float32)
    want = (x.astype(np.int64) @ _sylvester(256).T).astype(np.float64) / 16.0
    np.testing.assert_array_equal(O.kv4_fwht(x), want.astype(np.float32))
    e = np.eye(256, dtype=np.float32)[[0, 1, 37, 255]]
    np.testing.assert_array_equal(O.kv4_fwht(e), (_sylvester(256)[[0, 1, 37, 255]] / 16.0).astype(np.float32))


def _f16_bits(x):
    return int(np.array(x, dtype=np.float32).astype(np.float16).view(np.uint16))


def test_kv4_quant_by_hand():
    # group 0: max 7 -> scale f16(1) = 1, inv 1: 7 -> 15, -7 -> 1, 3.5 -> rint 4 (ties to even) -> 12, 2.5 -> 2
    # -> 10, -0.5 -> -0 -> 8, 0.49 -> 8. Byte i = value 2i (low nibble) | value 2i + 1 << 4.
    row = np.zeros(256, np.float32)
    row[:6] = [7, -7, 3.5, 2.5, -0.5, 0.49]
    # group 1 (values 32..63): max 1 -> dh = f16(1/7) = 0.142822265625 (rounded down), inv = 7.0017...:
    # 0.3571 * inv = 2.5003 -> 3, where an unrounded scale (inv = 7) gives 2.4997 -> 2
    row[32], row[33] = 1.0, 0.3571
    # group 2: all zero -> scale 0, inv 0, every value stored as 8
    # group 3: a max whose /7 falls below f16's smallest subnormal -> scale 0 -> every value 8
    row[96], row[97] = 1e-9, -1e-9
    # group 4: -3 max -> dh = f16(3/7) = 0.428466796875 (rounded down), inv = 2.33390: -3 -> -7.0017 -> -7 (nibble
    # 1), 1.5 -> 3.5009 -> 4 (nibble 12)
    row[128], row[129] = -3.0, 1.5
    q, sc = O.kv4_quant(row[None, :])
    q, sc = q[0], sc[0]
    assert list(q[:3]) == [15 | (1 << 4), 12 | (10 << 4), 8 | (8 << 4)]
    assert sc[0] == _f16_bits(1.0)
    assert sc[1] == _f16_bits(1.0 / 7.0) == 0x3092
    assert q[16] == 15 | (11 << 4)
    assert sc[2] == 0 and np.all(q[32:48] == 0x88)
    assert sc[3] == 0 and np.all(q[48:64] == 0x88)
    assert sc[4] == _f16_bits(np.float32(3.0) / np.float32(7.0))
    assert sc[4] == 0x36DB and q[64] == 1 | (12 << 4)
    assert np.all(q[65:] == 0x88) and np.all(q[3:16] == 0x88)


def test_kv4_quant_error_bound_and_dequant_order():
    # every dequantised value is within half a step (plus the f16 rounding) of the input, the nibble order is
    # value 2i low / 2i + 1 high, and each group of 32 has its own scale
    x = np.random.default_rng(2).standard_normal((40, 256)).astype(np.float32) * np.repeat(
        np.random.default_rng(3).uniform(0.1, 3, (40, 8)), 32, axis=1).astype(np.float32)
    q, sc = O.kv4_quant(x)
    deq = O.kv4_dequant(q, sc, 1).view(np.float16).astype(np.float64)
    step = np.repeat(sc.view(np.float16).astype(np.float64), 32, axis=1)
    assert np.all(np.abs(deq - x) <= 0.5 * step + np.abs(x) * 2.0 ** -10 + 1e-7)
    from attn_common import dequant_q4
    np.testing.assert_array_equal(deq, dequant_q4(q, sc, 1))


def test_rope_q4_rotates_q_and_k_and_quantises_the_rotated_rows():
    # the KV4 build's qk_norm_rope = the f16 build's qk_norm_rope, then kv4_fwht of every q and k head; the cache
    # holds kv4_quant of the rotated k rows and of the rotated v rows
    n, H, K, pos0, ctx = 5, 4, 2, 9, 16
    rng = np.random.default_rng(4)
    qkv = rng.standard_normal((n, (H + 2 * K) * 256)).astype(np.float32)
    qn = rng.uniform(0.5, 1.5, 256).astype(np.float32)
    kn = rng.uniform(0.5, 1.5, 256).astype(np.float32)
    z8 = np.zeros((ctx, K * 128), np.uint8)
    z16 = np.zeros((ctx, K * 8), np.uint16)
    got, kc, vc, ks, vs = O.qk_norm_rope_q4(qkv, z8, z8, z16, z16, pos0, H, K, qn=qn, kn=kn)
    f16c = np.zeros((ctx, K * 256), np.uint16)
    plain, _, _ = O.qk_norm_rope(qkv, f16c, f16c, pos0, H, K, hd=256, qn=qn, kn=kn)
    qk = plain[:, :(H + K) * 256].reshape(n * (H + K), 256)
    np.testing.assert_array_equal(got[:, :(H + K) * 256], O.kv4_fwht(qk).reshape(n, -1))
    np.testing.assert_array_equal(got[:, (H + K) * 256:], qkv[:, (H + K) * 256:])  # v heads pass unchanged
    kq, ksq = O.kv4_quant(got[:, H * 256:(H + K) * 256].reshape(n * K, 256))
    vq, vsq = O.kv4_quant(O.kv4_fwht(qkv[:, (H + K) * 256:].reshape(n * K, 256)))
    np.testing.assert_array_equal(kc[pos0:pos0 + n], kq.reshape(n, -1))
    np.testing.assert_array_equal(ks[pos0:pos0 + n], ksq.reshape(n, -1))
    np.testing.assert_array_equal(vc[pos0:pos0 + n], vq.reshape(n, -1))
    np.testing.assert_array_equal(vs[pos0:pos0 + n], vsq.reshape(n, -1))
    assert not kc[:pos0].any() and not vs[pos0 + n:].any()


def _q4_of_ints(ints, n_kv):
    """A 4-bit cache holding the integers `ints` (-7..7, [rows, n_kv*256]) with unit scales."""
    n = (ints.astype(np.int32) + 8).astype(np.uint8)
    return (n[:, 0::2] | (n[:, 1::2] << 4)).astype(np.uint8), np.full((ints.shape[0], n_kv * 8), 0x3C00, np.uint16)


def test_decode_tc256_q4_unit_scales_equal_the_int8_path():
    # integer values with unit scales: the 4-bit cache's f16 values are the integers themselves, so the KV4
    # decode equals the KV8 decode (pinned by hand above) with int8 rows of those integers and scales 1, bit for bit
    H, K, pos0, m = 16, 2, 700, 3
    rng = np.random.default_rng(8)
    q = rng.standard_normal((m, H * 256)).astype(np.float32)
    ki = rng.integers(-7, 8, (pos0 + m, K * 256)).astype(np.int8)
    vi = rng.integers(-7, 8, (pos0 + m, K * 256)).astype(np.int8)
    kc, ks = _q4_of_ints(ki, K)
    vc, vs = _q4_of_ints(vi, K)
    ones = np.ones((pos0 + m, K), np.float32)
    got = O.decode_tc256_q4(q, kc, vc, ks, vs, pos0, H, K)
    want = O.decode_tc256_i8(q, ki, vi, ones, ones, pos0, H, K)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("n_tok,pos0,n_heads,n_kv", [(1, 5, 16, 2), (1, 300, 16, 2), (8, 2000, 16, 2), (3, 77, 8, 1)])
def test_decode_tc256_q4_within_parity_bar(n_tok, pos0, n_heads, n_kv):
    q, kc, vc, ks, vs = make_inputs_q4(131 + pos0, n_tok, pos0 + n_tok, n_heads, n_kv)
    got = O.decode_tc256_q4(q, kc, vc, ks, vs, pos0, n_heads, n_kv)
    want = reference_f64_q4(q, kc, vc, ks, vs, pos0, n_heads, n_kv)
    ma, _ = assert_close(got, want, what="decode_tc256 KV4 semantics vs f64")
    assert ma > 1e-6


def test_decode_q4_rotation_gives_the_unrotated_attention():
    # rows rotated, quantised, attended with rotated queries and the output rotated back: the attention of the
    # original rows, to within the 4-bit rounding (closed form: one position gives its V row back)
    H, K, n = 8, 1, 200
    rng = np.random.default_rng(12)
    q = rng.standard_normal((1, H * 256)).astype(np.float32)
    k = rng.standard_normal((n, K * 256)).astype(np.float32)
    v = rng.standard_normal((n, K * 256)).astype(np.float32)
    kc, ks = O.kv4_quant(O.kv4_fwht(k.reshape(-1, 256)))
    vc, vs = O.kv4_quant(O.kv4_fwht(v.reshape(-1, 256)))
    qr = O.kv4_fwht(q.reshape(-1, 256)).reshape(1, -1)
    out = O.decode_tc256_q4(qr, kc.reshape(n, -1), vc.reshape(n, -1), ks.reshape(n, -1), vs.reshape(n, -1), n - 1, H, K)
    back = O.kv4_fwht(out.reshape(-1, 256)).reshape(1, -1)
    exact = _reference_f64_plain(q, k, v, n - 1, H, K)
    ma, _ = errors(back, exact)
    assert ma < 0.1  # 4-bit rows: about 2^-4 of the value range
    one = O.decode_tc256_q4(qr, kc.reshape(n, -1)[:1], vc.reshape(n, -1)[:1], ks.reshape(n, -1)[:1],
                            vs.reshape(n, -1)[:1], 0, H, K)
    v0 = O.kv4_dequant(vc.reshape(n, -1)[:1], vs.reshape(n, -1)[:1], K).view(np.float16).astype(np.float32)
    np.testing.assert_array_equal(one.reshape(H, 256), np.broadcast_to(v0, (H, 256)))


def _reference_f64_plain(q, k, v, pos0, n_heads, n_kv):
    from attn_common import _reference_f64_values
    return _reference_f64_values(q, k, v, pos0, n_heads, n_kv, 256)


def test_prefill_tc256_q4_unit_scales_equal_the_f16_path():
    # integer values with unit scales: the KV4 prefill stages exactly the f16 cache holding those integers
    H, K, pos0, n = 4, 2, 40, 70
    rng = np.random.default_rng(9)
    q = rng.standard_normal((n, H * 256)).astype(np.float32)
    ki = rng.integers(-7, 8, (pos0 + n, K * 256))
    vi = rng.integers(-7, 8, (pos0 + n, K * 256))
    kc, ks = _q4_of_ints(ki, K)
    vc, vs = _q4_of_ints(vi, K)
    got = O.prefill_tc256_q4(q, kc, vc, ks, vs, pos0, H, K)
    want = O.prefill_tc_semantics(q, ki.astype(np.float16).view(np.uint16), vi.astype(np.float16).view(np.uint16),
                                  pos0, H, K, hd=256)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("n,pos0,n_heads,n_kv", [(48, 0, 4, 2), (70, 33, 8, 1)])
def test_prefill_tc256_q4_within_parity_bar(n, pos0, n_heads, n_kv):
    q, kc, vc, ks, vs = make_inputs_q4(77 + n, n, pos0 + n, n_heads, n_kv)
    got = O.prefill_tc256_q4(q, kc, vc, ks, vs, pos0, n_heads, n_kv)
    want = reference_f64_q4(q, kc, vc, ks, vs, pos0, n_heads, n_kv)
    ma, _ = assert_close(got, want, what="prefill_tc256 KV4 semantics vs f64")
    assert ma > 1e-6


@pytest.mark.parametrize("n,pos0,n_heads,n_kv", [(48, 0, 4, 2), (70, 33, 4, 1)])
def test_prefill_tc_semantics_i8_hd256_within_parity_bar(n, pos0, n_heads, n_kv):
    # attention_prefill_tc256 with KV8: the int8 roundings at head size 256, within the bar of the exact attention
    q, k, v, ks, vs = make_inputs_i8(61 + n, n, pos0 + n, n_heads, n_kv, hd=256)
    got = O.prefill_tc_semantics_i8(q, k, v, ks, vs, pos0, n_heads, n_kv, hd=256)
    ma, _ = assert_close(got, reference_f64_i8(q, k, v, ks, vs, pos0, n_heads, n_kv, hd=256),
                         what="int8 prefill hd256 semantics vs f64")
    assert ma > 1e-6


def test_prefill_i8_hd256_unit_scales_follow_the_f16_path():
    q, k, v, _, _ = make_inputs_i8(9, 50, 120, 4, 2, hd=256)
    k = (k // 16).astype(np.int8)
    ones = np.ones((120, 2), dtype=np.float32)
    got = O.prefill_tc_semantics_i8(q, k, v, ones, ones, 70, 4, 2, hd=256)
    want = O.prefill_tc_semantics(q, k.astype(np.float16).view(np.uint16), v.astype(np.float16).view(np.uint16), 70,
                                  4, 2, hd=256)
    np.testing.assert_allclose(got, want, rtol=0, atol=1e-4)
