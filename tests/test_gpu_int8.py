"""Parity of the int8 KV cache path (the reference's KV8 build: kv_store src/cuda.rs:333-339, decode
src/cuda.rs:1684-1865 + 2806-2836) on the gfx950 kernels, through the C ABI.

Bar: max-abs 2e-3 and relative L2 1e-3 against the oracle's restatement of the reference's int8 decode,
and 2e-5 against float64 attention over the dequantised cache (the kernels widen int8 exactly and keep
f32 scores). The cache write is checked against the oracle's quantiser: V rows (copied, not rotated)
byte for byte with equal scales; K rows (after RoPE, whose angles differ by an ulp between sin/cos
implementations) within one quantisation step plus the f32 tolerance.
"""
import sys

import numpy as np
import pytest
import torch

import gi_attn
import gi_oracle as O
from attn_common import assert_close, make_inputs_i8, reference_f64_i8

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


def to_dev_i8(q, k, v, ks, vs, dev, layout="reference", n_kv=None):
    qt = torch.from_numpy(np.ascontiguousarray(q)).to(dev)
    if layout == "head_major":
        k = np.ascontiguousarray(k.reshape(k.shape[0], n_kv, -1).transpose(1, 0, 2))
        v = np.ascontiguousarray(v.reshape(v.shape[0], n_kv, -1).transpose(1, 0, 2))
        ks, vs = np.ascontiguousarray(ks.T), np.ascontiguousarray(vs.T)
    return (qt, torch.from_numpy(np.ascontiguousarray(k)).to(dev), torch.from_numpy(np.ascontiguousarray(v)).to(dev),
            torch.from_numpy(np.ascontiguousarray(ks)).to(dev), torch.from_numpy(np.ascontiguousarray(vs)).to(dev))


def run_decode_i8(q, k, v, ks, vs, pos0, n_heads, n_kv, dev, layout="reference", **kw):
    qt, kt, vt, kst, vst = to_dev_i8(q, k, v, ks, vs, dev, layout, n_kv)
    out = gi_attn.decode(qt, kt, vt, pos0, n_heads, n_kv, k_scale=kst, v_scale=vst, kv_layout=layout, **kw)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def check(got, q, k, v, ks, vs, pos0, n_heads, n_kv, what):
    assert_close(got, O.decode_gpu_semantics_i8(q, k, v, ks, vs, pos0, n_heads, n_kv), what=f"{what} vs oracle")
    assert_close(got, reference_f64_i8(q, k, v, ks, vs, pos0, n_heads, n_kv), max_abs=2e-5, rel_l2=2e-5,
                 what=f"{what} vs f64")


def test_decode_i8_graph_replay(gpu):
    # an 8-token verify block over the int8 cache with a device position, captured once and replayed at
    # several positions with eager work between the replays
    n_tok, n_heads, n_kv, cap = 8, 32, 4, 3000
    q, k, v, ks, vs = make_inputs_i8(93, n_tok, cap, n_heads, n_kv)
    qt, kt, vt, kst, vst = to_dev_i8(q, k, v, ks, vs, gpu)
    ws = gi_attn.new_workspace(cap, n_tok, n_heads, n_kv, device=gpu)
    posp = torch.zeros(1, dtype=torch.int32, device=gpu)
    out = torch.zeros((n_tok, n_heads * 128), dtype=torch.float32, device=gpu)
    kw = dict(out=out, workspace=ws, posp=posp, ctx_cap=cap, k_scale=kst, v_scale=vst)
    gi_attn.decode(qt, kt, vt, 0, n_heads, n_kv, **kw)  # warm-up
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        gi_attn.decode(qt, kt, vt, 0, n_heads, n_kv, **kw)
    for pos in (cap - n_tok, 40, 1500, 0):
        say("decode i8 graph replay", pos)
        posp.fill_(pos)
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert_close(out.cpu().numpy(), reference_f64_i8(q, k, v, ks, vs, pos, n_heads, n_kv), max_abs=2e-5,
                     rel_l2=2e-5, what=f"i8 replay at {pos}")


DECODE_SHAPES_I8 = [
    # (n_tok, pos0, n_heads, n_kv): spans inside one tile, at tile and slice edges, verify blocks of every
    # kernel variant (1 and 2 column blocks, one to four pair groups), G = 3 and 6 pair layouts
    (1, 0, 32, 8),
    (1, 63, 32, 4),
    (1, 64, 32, 4),
    (1, 255, 8, 8),
    (1, 256, 32, 4),
    (1, 1000, 32, 4),
    (1, 4095, 32, 8),
    (2, 300, 32, 4),
    (3, 60, 16, 2),
    (8, 200, 32, 4),
    (15, 513, 32, 8),
    (5, 77, 12, 4),
    (4, 40, 6, 1),
    (2, 63, 32, 4),  # wave 1's first tile (keys 64..) lies past token 0's span but not token 1's
    (15, 700, 32, 4),  # 120 pairs per kv head: one pair per column, four workgroups per (slice, kv head)
    (4, 1000, 32, 4),  # 32 pairs: two full column blocks per wave
    (6, 130, 32, 4),   # 48 pairs: two workgroups per (slice, kv head), the second half idle
    (4, 40, 16, 1),    # 64 pairs on one kv head, one slice: fewer (slice, kv head) items than XCDs
    (16, 1000, 32, 4),  # 128 pairs: two pair sets of 32 per workgroup, two workgroups per (slice, kv head)
    (32, 513, 32, 4),   # 256 pairs: the same layout, four workgroups
    (8, 2500, 64, 4),   # 128 pairs at G = 16, a span of several slices
    (8, 249, 32, 4),  # token 0's span ends before the last slice: its partial there is empty (m = -inf) and the merge skips it
    (2, 255, 8, 2),    # the same with 8 pairs: token 0 sees all of slice 0 and none of slice 1
]


@pytest.mark.parametrize("n_tok,pos0,n_heads,n_kv", DECODE_SHAPES_I8)
def test_decode_i8_small(gpu, n_tok, pos0, n_heads, n_kv):
    say("decode i8", n_tok, pos0, n_heads, n_kv)
    q, k, v, ks, vs = make_inputs_i8(5000 + pos0, n_tok, pos0 + n_tok, n_heads, n_kv)
    got = run_decode_i8(q, k, v, ks, vs, pos0, n_heads, n_kv, gpu)
    check(got, q, k, v, ks, vs, pos0, n_heads, n_kv, "decode i8")


def test_decode_i8_ctx65536(gpu):
    say("decode i8 ctx 65536 32q/4kv")
    q, k, v, ks, vs = make_inputs_i8(6, 1, 65536, 32, 4)
    got = run_decode_i8(q, k, v, ks, vs, 65535, 32, 4, gpu)
    check(got, q, k, v, ks, vs, 65535, 32, 4, "decode i8 C2 shape")


def test_verify_i8_8tok_at_32768(gpu):
    say("verify i8 8 tokens @ 32768 32q/4kv")
    q, k, v, ks, vs = make_inputs_i8(7, 8, 32776, 32, 4)
    got = run_decode_i8(q, k, v, ks, vs, 32768, 32, 4, gpu)
    check(got, q, k, v, ks, vs, 32768, 32, 4, "verify i8 C4 shape")


@pytest.mark.parametrize("n_tok,pos0,n_heads,n_kv", [(1, 300, 32, 4), (1, 65535, 32, 4), (8, 1000, 32, 4),
                                                    (16, 4000, 32, 4)])
def test_decode_i8_head_major(gpu, n_tok, pos0, n_heads, n_kv):
    say("decode i8 head-major", n_tok, pos0, n_heads, n_kv)
    q, k, v, ks, vs = make_inputs_i8(7000 + pos0, n_tok, pos0 + n_tok, n_heads, n_kv)
    got = run_decode_i8(q, k, v, ks, vs, pos0, n_heads, n_kv, gpu, layout="head_major")
    check(got, q, k, v, ks, vs, pos0, n_heads, n_kv, "decode i8 head-major")


def test_decode_i8_zero_scale_rows(gpu):
    # rows whose scale is 0 (an all-zero row as kv_store writes it) score 0 and weigh nothing in V
    q, k, v, ks, vs = make_inputs_i8(71, 1, 700, 32, 4)
    ks[100:164] = 0
    vs[300:310] = 0
    k[100:164] = 0
    v[300:310] = 0
    say("decode i8 zero-scale rows")
    got = run_decode_i8(q, k, v, ks, vs, 699, 32, 4, gpu)
    check(got, q, k, v, ks, vs, 699, 32, 4, "decode i8 zero rows")


def test_decode_i8_device_position(gpu):
    n_heads, n_kv, cap = 32, 4, 3000
    q, k, v, ks, vs = make_inputs_i8(78, 1, cap, n_heads, n_kv)
    qt, kt, vt, kst, vst = to_dev_i8(q, k, v, ks, vs, gpu)
    ws = gi_attn.new_workspace(cap, 1, n_heads, n_kv, device=gpu)
    posp = torch.zeros(1, dtype=torch.int32, device=gpu)
    for pos in (0, 64, 1999, 2999):
        say("decode i8 posp", pos)
        posp.fill_(pos)
        out = gi_attn.decode(qt, kt, vt, 99999, n_heads, n_kv, k_scale=kst, v_scale=vst, workspace=ws, posp=posp,
                             ctx_cap=cap)
        torch.cuda.synchronize()
        assert_close(out.cpu().numpy(), reference_f64_i8(q, k, v, ks, vs, pos, n_heads, n_kv), max_abs=2e-5,
                     rel_l2=2e-5, what=f"i8 posp {pos}")


def test_decode_i8_and_f16_share_a_workspace(gpu):
    # calls of both cache types through one workspace, in turn: each matches its own reference
    from attn_common import make_inputs, reference_f64
    n_heads, n_kv, cap = 32, 4, 5000
    ws = gi_attn.new_workspace(cap, 15, n_heads, n_kv, device=gpu)
    for i, (n_tok, pos0) in enumerate(((1, 4999), (15, 100), (8, 3000), (1, 200))):
        say("decode i8/f16 shared workspace", n_tok, pos0)
        q, k, v, ks, vs = make_inputs_i8(900 + i, n_tok, pos0 + n_tok, n_heads, n_kv)
        got = run_decode_i8(q, k, v, ks, vs, pos0, n_heads, n_kv, gpu, workspace=ws)
        assert_close(got, reference_f64_i8(q, k, v, ks, vs, pos0, n_heads, n_kv), max_abs=2e-5, rel_l2=2e-5,
                     what=f"i8 {n_tok}@{pos0}")
        q, kb, vb = make_inputs(950 + i, n_tok, pos0 + n_tok, n_heads, n_kv)
        qt = torch.from_numpy(q).to(gpu)
        kt = torch.from_numpy(kb.view(np.int16)).to(gpu).view(torch.float16)
        vt = torch.from_numpy(vb.view(np.int16)).to(gpu).view(torch.float16)
        out = gi_attn.decode(qt, kt, vt, pos0, n_heads, n_kv, workspace=ws)
        torch.cuda.synchronize()
        assert_close(out.cpu().numpy(), reference_f64(q, kb, vb, pos0, n_heads, n_kv), max_abs=2e-5, rel_l2=2e-5,
                     what=f"f16 {n_tok}@{pos0}")


# ---------------------------------------------------------------- cache write (qk_norm_rope with KV8)

ROPE_I8_SHAPES = [
    # (n, pos0, n_heads, n_kv, hd, neox, norm, layout)
    (1, 4095, 32, 8, 128, True, True, "reference"),
    (7, 100, 16, 4, 64, False, False, "reference"),
    (300, 0, 32, 4, 128, True, True, "head_major"),
    (3, 2000, 8, 2, 256, True, True, "reference"),
    (5, 300, 12, 4, 96, True, True, "reference"),   # a head size of the f32 kernels (the lane-masked store)
    (33, 40, 32, 32, 80, False, True, "head_major"),
]
# seeded random shapes: head sizes 64/128/256, 1-300 rows at positions up to 5000, 1-8 kv heads, group sizes 1-8
_rng = np.random.default_rng(51)
for _ in range(8):
    _kv = int(_rng.choice([1, 2, 4, 8]))
    ROPE_I8_SHAPES.append((int(_rng.integers(1, 301)), int(_rng.integers(0, 5001)), _kv * int(_rng.integers(1, 9)), _kv,
                           int(_rng.choice([64, 128, 256])), bool(_rng.integers(0, 2)), bool(_rng.integers(0, 2)),
                           str(_rng.choice(["reference", "head_major"]))))


@pytest.mark.parametrize("n,pos0,n_heads,n_kv,hd,neox,norm,layout", ROPE_I8_SHAPES)
def test_qk_norm_rope_i8_matches_oracle(gpu, n, pos0, n_heads, n_kv, hd, neox, norm, layout):
    say("qk_norm_rope i8", n, pos0, n_heads, n_kv, hd, neox, norm, layout)
    rng = np.random.default_rng(900 + n)
    qkv = rng.standard_normal((n, (n_heads + 2 * n_kv) * hd), dtype=np.float32)
    qkv[0, (n_heads + n_kv) * hd:(n_heads + n_kv + 1) * hd] = 0  # a zero v row: scale 0, zero bytes
    cap = pos0 + n + 5
    kc = np.full((cap, n_kv * hd), 99, dtype=np.int8)
    sc = np.full((cap, n_kv), -1.0, dtype=np.float32)
    qn = rng.uniform(0.5, 1.5, hd).astype(np.float32) if norm else None
    kn = rng.uniform(0.5, 1.5, hd).astype(np.float32) if norm else None
    want, wk, wv, wks, wvs = O.qk_norm_rope_i8(qkv, kc, kc, sc, sc, pos0, n_heads, n_kv, hd=hd, base=1e6, qn=qn,
                                               kn=kn, neox=neox)
    dev = lambda a: None if a is None else torch.from_numpy(np.ascontiguousarray(a)).to(gpu)
    qt = dev(qkv)
    kt, vt = dev(kc.reshape(cap, n_kv, hd)), dev(kc.reshape(cap, n_kv, hd))
    kst, vst = dev(sc), dev(sc)
    if layout == "head_major":
        kt, vt = kt.transpose(0, 1).contiguous(), vt.transpose(0, 1).contiguous()
        kst, vst = kst.t().contiguous(), vst.t().contiguous()
    gi_attn.qk_norm_rope(qt, kt, vt, pos0, n_heads, n_kv, hd=hd, base=1e6, qn=dev(qn), kn=dev(kn), neox=neox,
                         kv_layout=layout, k_scale=kst, v_scale=vst)
    torch.cuda.synchronize()
    if layout == "head_major":
        kt, vt = kt.transpose(0, 1).contiguous(), vt.transpose(0, 1).contiguous()
        kst, vst = kst.t().contiguous(), vst.t().contiguous()
    got = qt.cpu().numpy()
    gk, gv = kt.cpu().numpy().reshape(cap, -1), vt.cpu().numpy().reshape(cap, -1)
    gks, gvs = kst.cpu().numpy(), vst.cpu().numpy()
    assert np.abs(got - want).max() <= 2e-3
    # V: the input rows quantised, bit for bit (including the zero row's scale 0)
    np.testing.assert_array_equal(gv, wv)
    np.testing.assert_array_equal(gvs, wvs)
    assert gvs[pos0, 0] == 0
    # K: dequantised values within one step of the oracle's plus the rotation tolerance
    rows = slice(pos0, pos0 + n)
    gkd = gk[rows].reshape(n, n_kv, hd).astype(np.float64) * gks[rows][:, :, None]
    wkd = wk[rows].reshape(n, n_kv, hd).astype(np.float64) * wks[rows][:, :, None]
    assert np.all(np.abs(gkd - wkd) <= 2e-3 + wks[rows][:, :, None] * 1.0001)
    np.testing.assert_allclose(gks[rows], wks[rows], rtol=2e-3, atol=2e-5)
    other = np.r_[0:pos0, pos0 + n:cap]
    assert np.all(gk[other] == 99) and np.all(gv[other] == 99)
    assert np.all(gks[other] == -1) and np.all(gvs[other] == -1)


def test_qk_norm_rope_i8_then_decode_matches_the_oracle_pipeline(gpu):
    # store a new token's K/V into an int8 cache, then decode over it, against the oracle doing both
    n_heads, n_kv, hd, pos = 32, 4, 128, 2500
    _, kc, vc, ks, vs = make_inputs_i8(812, 1, pos + 1, n_heads, n_kv)
    rng = np.random.default_rng(813)
    qkv = rng.standard_normal((1, (n_heads + 2 * n_kv) * hd), dtype=np.float32)
    qn = rng.uniform(0.5, 1.5, hd).astype(np.float32)
    kn = rng.uniform(0.5, 1.5, hd).astype(np.float32)
    o_qkv, o_kc, o_vc, o_ks, o_vs = O.qk_norm_rope_i8(qkv, kc, vc, ks, vs, pos, n_heads, n_kv, qn=qn, kn=kn, base=1e6)
    want = O.decode_gpu_semantics_i8(o_qkv[:, :n_heads * hd], o_kc, o_vc, o_ks, o_vs, pos, n_heads, n_kv)
    say("qk_norm_rope i8 + decode i8")
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)
    qt, kt, vt, kst, vst = dev(qkv), dev(kc), dev(vc), dev(ks), dev(vs)
    gi_attn.qk_norm_rope(qt, kt, vt, pos, n_heads, n_kv, qn=dev(qn), kn=dev(kn), base=1e6, k_scale=kst, v_scale=vst)
    out = gi_attn.decode(qt[:, :n_heads * hd], kt, vt, pos, n_heads, n_kv, k_scale=kst, v_scale=vst)
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), want, what="qk_norm_rope i8 + decode i8 vs oracle")


# ---------------------------------------------------------------- prefill (attention_prefill_tc with KV8)

PREFILL_I8_SHAPES = [
    # (n, pos0, n_heads, n_kv, q dtype, out dtype, layout): tile and diagonal edges, chunks at a prefix,
    # partial last tiles, both layouts
    (16, 0, 8, 2, np.float16, torch.float32, "reference"),
    (64, 0, 8, 2, np.float32, torch.float32, "reference"),
    (129, 0, 8, 8, np.float16, torch.float32, "reference"),
    (300, 0, 32, 4, np.float32, torch.float32, "head_major"),
    (70, 130, 8, 4, np.float16, torch.float32, "reference"),
    (256, 256, 32, 4, np.float16, torch.float16, "head_major"),
    (1000, 24, 16, 2, np.float16, torch.float32, "reference"),
]


def run_prefill_i8(q, k, v, ks, vs, pos0, n_heads, n_kv, dev, layout="reference", out_dtype=torch.float32):
    qt, kt, vt, kst, vst = to_dev_i8(q, k, v, ks, vs, dev, layout, n_kv)
    out = gi_attn.prefill(qt, kt, vt, pos0, n_heads, n_kv, out_dtype=out_dtype, kv_layout=layout, k_scale=kst,
                          v_scale=vst)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


@pytest.mark.parametrize("n,pos0,n_heads,n_kv,qd,od,layout", PREFILL_I8_SHAPES)
def test_prefill_i8_small(gpu, n, pos0, n_heads, n_kv, qd, od, layout):
    say("prefill i8", n, pos0, n_heads, n_kv, qd.__name__, od, layout)
    q, k, v, ks, vs = make_inputs_i8(8000 + n + pos0, n, pos0 + n, n_heads, n_kv)
    q = q.astype(qd)
    got = run_prefill_i8(q, k, v, ks, vs, pos0, n_heads, n_kv, gpu, layout, od)
    q32 = q.astype(np.float32)
    assert_close(got, O.prefill_tc_semantics_i8(q32, k, v, ks, vs, pos0, n_heads, n_kv),
                 what="prefill i8 vs oracle (reference int8 prefill semantics)")
    assert_close(got, reference_f64_i8(q32, k, v, ks, vs, pos0, n_heads, n_kv), what="prefill i8 vs f64")


def test_prefill_i8_8192(gpu):
    # config 3's shape over an int8 cache: the whole output against a torch fp32 reference over the
    # dequantised cache (on the GPU), sampled rows against the float64 reference
    n, n_heads, n_kv = 8192, 32, 8
    say("prefill i8 8192 32q/8kv")
    q, k, v, ks, vs = make_inputs_i8(9, n, n, n_heads, n_kv)
    q = q.astype(np.float16)
    qt, kt, vt, kst, vst = to_dev_i8(q, k, v, ks, vs, gpu)
    out = gi_attn.prefill(qt, kt, vt, 0, n_heads, n_kv, out_dtype=torch.float16, k_scale=kst, v_scale=vst)
    kd = (kt.view(n, n_kv, 128).float() * kst[:, :, None]).view(n, -1)
    vd = (vt.view(n, n_kv, 128).float() * vst[:, :, None]).view(n, -1)
    G = n_heads // n_kv
    Q = qt.view(n, n_heads, 128).float()
    K, V = kd.view(n, n_kv, 128), vd.view(n, n_kv, 128)
    mask = torch.arange(n, device=gpu)[None, :] > torch.arange(n, device=gpu)[:, None]
    ref = torch.empty((n, n_heads, 128), dtype=torch.float32, device=gpu)
    for h in range(n_heads):
        s = (Q[:, h] @ K[:, h // G].T) / 128 ** 0.5
        s.masked_fill_(mask, float("-inf"))
        ref[:, h] = torch.softmax(s, dim=-1) @ V[:, h // G]
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    assert_close(got, ref.view(n, -1).cpu().numpy(), what="prefill i8 8192 vs torch fp32")
    for r in (0, 63, 64, 1000, 8191):
        assert_close(got[r:r + 1], reference_f64_i8(q[r:r + 1].astype(np.float32), k, v, ks, vs, r, n_heads, n_kv),
                     what=f"prefill i8 row {r} vs f64")


@pytest.mark.parametrize("n,pos0,exact", [(1, 99, False), (8, 300, True), (20, 0, False), (40, 17, True)])
def test_attention_operator_i8(gpu, n, pos0, exact):
    # GpuModel::attention over the int8 cache: prefill for >= 16 tokens unless exact, the split path otherwise
    say("operator i8", n, pos0, exact)
    n_heads, n_kv, hd = 32, 8, 128
    row = n_heads * hd + 2 * n_kv * hd
    qkv = np.random.default_rng(95 + n).standard_normal((n, row), dtype=np.float32)
    _, k, v, ks, vs = make_inputs_i8(96 + n, 1, pos0 + n, n_heads, n_kv)
    qkv_t = torch.from_numpy(qkv).to(gpu)
    _, kt, vt, kst, vst = to_dev_i8(qkv[:, :1], k, v, ks, vs, gpu)
    out = gi_attn.attention(qkv_t, kt, vt, pos0, n_heads, n_kv, exact=exact, k_scale=kst, v_scale=vst)
    torch.cuda.synchronize()
    q = np.ascontiguousarray(qkv[:, :n_heads * hd])
    split_path = n < 16 or exact
    assert_close(out.cpu().numpy(), reference_f64_i8(q, k, v, ks, vs, pos0, n_heads, n_kv),
                 max_abs=2e-5 if split_path else 2e-3, rel_l2=2e-5 if split_path else 1e-3, what="operator i8 vs f64")
