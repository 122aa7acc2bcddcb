"""Parity of head size 256 (the reference's wide heads, src/cuda.rs:1762-1781 and attention_prefill_tc256
src/cuda.rs:2623) on the gfx950 kernels, through the C ABI.

Bar: max-abs 2e-3 and relative L2 1e-3 against the oracle's Model::attention (src/model.rs:1320-1409, any
head size), and 2e-5 against float64 attention for decode over the f16 cache (f32 scores and probabilities, as
at head size 128). Decode over the int8 cache follows the reference's attention_decode_tc256 arithmetic (one f16
Q, one f16 P): within REF_ORACLE_TOL of the oracle's restatement of it and within the bar of float64.
"""
import sys

import numpy as np
import pytest
import torch

import gi_attn
import gi_oracle as O
from attn_common import (REF_ORACLE_TOL, assert_close, make_inputs, make_inputs_i8, reference_f64, reference_f64_i8,
                         split_f64_tol)

pytestmark = pytest.mark.gpu
HD = 256


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


def to_dev(q, k, v, dev, n_kv, layout="reference"):
    qt = torch.from_numpy(np.ascontiguousarray(q)).to(dev)
    kt = torch.from_numpy(np.ascontiguousarray(k).view(np.int16)).to(dev).view(torch.float16)
    vt = torch.from_numpy(np.ascontiguousarray(v).view(np.int16)).to(dev).view(torch.float16)
    if layout == "head_major":
        kt = kt.view(-1, n_kv, HD).transpose(0, 1).contiguous()
        vt = vt.view(-1, n_kv, HD).transpose(0, 1).contiguous()
    return qt, kt, vt


DECODE_SHAPES_256 = [
    # (n_tok, pos0, n_heads, n_kv): spans inside one 16-key tile, at tile and slice edges, every kernel
    # variant (up to 8 pairs: 1 and 2 column blocks; above: one pair per column, two pair sets per workgroup), G = 3
    (1, 0, 16, 2),
    (1, 15, 16, 2),
    (1, 16, 32, 4),
    (1, 63, 16, 4),
    (1, 64, 16, 4),
    (1, 1000, 32, 4),
    (1, 4095, 16, 2),
    (2, 300, 16, 2),
    (8, 200, 32, 4),
    (15, 513, 16, 2),
    (5, 77, 12, 4),   # slice 1's second wave tile lies past token 0's span but not token 4's
    (2, 15, 16, 2),   # wave 1's first tile (keys 16..) lies past token 0's span but not token 1's
    (3, 60, 16, 2),   # 24 pairs: one pair per column, waves 2 and 3 idle
    (6, 130, 16, 2),  # 48 pairs
    (1, 3000, 32, 2), # G = 16: one token's 16 pairs, one pair per column
    (2, 2000, 32, 1), # G = 32, two tokens: 64 pairs on one kv head
    (8, 249, 16, 2),  # token 0's span ends before the last slice: its partial there is empty (m = -inf) and the merge skips it
    (2, 63, 16, 2),   # the same with 4 pairs: token 0 sees all of slice 0 and none of slice 1
]


@pytest.mark.parametrize("n_tok,pos0,n_heads,n_kv", DECODE_SHAPES_256)
def test_decode_hd256(gpu, n_tok, pos0, n_heads, n_kv):
    say("decode hd256", n_tok, pos0, n_heads, n_kv)
    q, k, v = make_inputs(6000 + pos0, n_tok, pos0 + n_tok, n_heads, n_kv, hd=HD)
    qt, kt, vt = to_dev(q, k, v, gpu, n_kv)
    out = gi_attn.decode(qt, kt, vt, pos0, n_heads, n_kv, hd=HD)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert_close(got, O.attention(q, k, v, pos0, n_heads, n_kv, hd=HD), what="decode hd256 vs oracle")
    assert_close(got, reference_f64(q, k, v, pos0, n_heads, n_kv, hd=HD), max_abs=2e-5, rel_l2=2e-5,
                 what="decode hd256 vs f64")


@pytest.mark.parametrize("layout", ["reference", "head_major"])
def test_decode_hd256_ctx65536(gpu, layout):
    # config 2's context with 256-wide heads (16 query / 2 kv heads: Qwen3.5-style)
    say("decode hd256 ctx 65536 16q/2kv", layout)
    q, k, v = make_inputs(61, 1, 65536, 16, 2, hd=HD)
    qt, kt, vt = to_dev(q, k, v, gpu, 2, layout)
    out = gi_attn.decode(qt, kt, vt, 65535, 16, 2, hd=HD, kv_layout=layout)
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), reference_f64(q, k, v, 65535, 16, 2, hd=HD), max_abs=2e-5, rel_l2=2e-5,
                 what="decode hd256 C2 context vs f64")


def test_decode_hd256_device_position(gpu):
    n_heads, n_kv, cap = 16, 2, 2000
    q, k, v = make_inputs(62, 1, cap, n_heads, n_kv, hd=HD)
    qt, kt, vt = to_dev(q, k, v, gpu, n_kv)
    ws = gi_attn.new_workspace(cap, 1, n_heads, n_kv, hd=HD, device=gpu)
    posp = torch.zeros(1, dtype=torch.int32, device=gpu)
    for pos in (0, 17, 1999):
        say("decode hd256 posp", pos)
        posp.fill_(pos)
        out = gi_attn.decode(qt, kt, vt, 12345, n_heads, n_kv, hd=HD, workspace=ws, posp=posp, ctx_cap=cap)
        torch.cuda.synchronize()
        assert_close(out.cpu().numpy(), reference_f64(q, k, v, pos, n_heads, n_kv, hd=HD), max_abs=2e-5,
                     rel_l2=2e-5, what=f"hd256 posp {pos}")


# ---------------------------------------------------------------- decode over the int8 cache (attention_decode_tc256)

def to_dev_i8(q, k, v, ks, vs, dev, n_kv, layout="reference"):
    if layout == "head_major":
        k = np.ascontiguousarray(k.reshape(k.shape[0], n_kv, HD).transpose(1, 0, 2))
        v = np.ascontiguousarray(v.reshape(v.shape[0], n_kv, HD).transpose(1, 0, 2))
        ks, vs = np.ascontiguousarray(ks.T), np.ascontiguousarray(vs.T)
    return [torch.from_numpy(np.ascontiguousarray(x)).to(dev) for x in (q, k, v, ks, vs)]


def check_i8(got, q, k, v, ks, vs, pos0, n_heads, n_kv, what, oracle=True):
    # the reference's tc256 rounds Q and P*vscale to f16, and so do these kernels
    if oracle:
        assert_close(got, O.decode_tc256_i8(q, k, v, ks, vs, pos0, n_heads, n_kv), *REF_ORACLE_TOL,
                     what=f"{what} vs oracle (tc256)")
    assert_close(got, reference_f64_i8(q, k, v, ks, vs, pos0, n_heads, n_kv, hd=HD), *split_f64_tol("i8", HD),
                 what=f"{what} vs f64")


@pytest.mark.parametrize("n_tok,pos0,n_heads,n_kv", DECODE_SHAPES_256)
def test_decode_hd256_i8(gpu, n_tok, pos0, n_heads, n_kv):
    say("decode hd256 i8", n_tok, pos0, n_heads, n_kv)
    q, k, v, ks, vs = make_inputs_i8(7000 + pos0, n_tok, pos0 + n_tok, n_heads, n_kv, hd=HD)
    qt, kt, vt, kst, vst = to_dev_i8(q, k, v, ks, vs, gpu, n_kv)
    out = gi_attn.decode(qt, kt, vt, pos0, n_heads, n_kv, hd=HD, k_scale=kst, v_scale=vst)
    torch.cuda.synchronize()
    check_i8(out.cpu().numpy(), q, k, v, ks, vs, pos0, n_heads, n_kv, "decode hd256 i8")


@pytest.mark.parametrize("n_tok,layout", [(1, "reference"), (1, "head_major"), (8, "head_major")])
def test_decode_hd256_i8_long_context(gpu, n_tok, layout):
    # 65536 keys (one token) and an 8-token verify block at a 32768-key prefix, 16 query / 2 kv heads
    ctx = 65536 if n_tok == 1 else 32768 + n_tok
    say("decode hd256 i8", ctx, n_tok, layout)
    q, k, v, ks, vs = make_inputs_i8(71 + n_tok, n_tok, ctx, 16, 2, hd=HD)
    qt, kt, vt, kst, vst = to_dev_i8(q, k, v, ks, vs, gpu, 2, layout)
    out = gi_attn.decode(qt, kt, vt, ctx - n_tok, 16, 2, hd=HD, k_scale=kst, v_scale=vst, kv_layout=layout)
    torch.cuda.synchronize()
    check_i8(out.cpu().numpy(), q, k, v, ks, vs, ctx - n_tok, 16, 2, f"hd256 i8 {ctx} keys", oracle=n_tok > 1)


def test_decode_hd256_i8_graph_replay(gpu):
    # an 8-token verify block (one pair per column, 32 pairs per workgroup) with a device position, captured once and
    # replayed at several positions with eager work between the replays
    n_tok, n_heads, n_kv, cap = 8, 16, 2, 2500
    q, k, v, ks, vs = make_inputs_i8(95, n_tok, cap, n_heads, n_kv, hd=HD)
    qt, kt, vt, kst, vst = to_dev_i8(q, k, v, ks, vs, gpu, n_kv)
    ws = gi_attn.new_workspace(cap, n_tok, n_heads, n_kv, hd=HD, device=gpu)
    posp = torch.zeros(1, dtype=torch.int32, device=gpu)
    out = torch.zeros((n_tok, n_heads * HD), dtype=torch.float32, device=gpu)
    kw = dict(hd=HD, out=out, workspace=ws, posp=posp, ctx_cap=cap, k_scale=kst, v_scale=vst)
    gi_attn.decode(qt, kt, vt, 0, n_heads, n_kv, **kw)  # warm-up
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        gi_attn.decode(qt, kt, vt, 0, n_heads, n_kv, **kw)
    for pos in (cap - n_tok, 31, 1000, 0):
        say("decode hd256 i8 graph replay", pos)
        posp.fill_(pos)
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        check_i8(out.cpu().numpy(), q, k, v, ks, vs, pos, n_heads, n_kv, f"hd256 i8 replay at {pos}")


# ---------------------------------------------------------------- prefill (attention_prefill_tc256)

PREFILL_SHAPES_256 = [
    # (n, pos0, n_heads, n_kv, q dtype, out dtype, layout): one tile, diagonal and tile edges (64 keys,
    # 128 query rows per workgroup), chunks at a prefix, both layouts
    (16, 0, 8, 2, np.float16, torch.float32, "reference"),
    (33, 0, 4, 1, np.float32, torch.float32, "reference"),
    (65, 0, 4, 1, np.float16, torch.float32, "reference"),
    (127, 63, 8, 2, np.float16, torch.float32, "head_major"),
    (128, 0, 16, 2, np.float16, torch.float16, "reference"),
    (129, 0, 8, 8, np.float16, torch.float32, "head_major"),
    (300, 40, 16, 2, np.float32, torch.float32, "reference"),
    (70, 130, 8, 4, np.float16, torch.float32, "head_major"),
    (1000, 24, 16, 2, np.float16, torch.float32, "reference"),
]


@pytest.mark.parametrize("n,pos0,n_heads,n_kv,qd,od,layout", PREFILL_SHAPES_256)
def test_prefill_hd256(gpu, n, pos0, n_heads, n_kv, qd, od, layout):
    say("prefill hd256", n, pos0, n_heads, n_kv, qd.__name__, od, layout)
    q, k, v = make_inputs(7000 + n + pos0, n, pos0 + n, n_heads, n_kv, hd=HD, q_dtype=qd)
    qt, kt, vt = to_dev(q, k, v, gpu, n_kv, layout)
    out = gi_attn.prefill(qt, kt, vt, pos0, n_heads, n_kv, hd=HD, out_dtype=od, kv_layout=layout)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    q32 = q.astype(np.float32)
    assert_close(got, O.prefill_tc_semantics(q32, k, v, pos0, n_heads, n_kv, hd=HD),
                 what="prefill hd256 vs oracle (attention_prefill_tc256 semantics)")
    assert_close(got, reference_f64(q32, k, v, pos0, n_heads, n_kv, hd=HD), what="prefill hd256 vs f64")


def test_prefill_hd256_4096(gpu):
    # a 4096-token prompt with 256-wide heads (16 query / 2 kv heads): the whole output against a torch fp32
    # reference on the GPU, sampled rows against float64
    n, n_heads, n_kv = 4096, 16, 2
    say("prefill hd256 4096 16q/2kv")
    q, k, v = make_inputs(71, n, n, n_heads, n_kv, hd=HD, q_dtype=np.float16)
    qt, kt, vt = to_dev(q, k, v, gpu, n_kv)
    out = gi_attn.prefill(qt, kt, vt, 0, n_heads, n_kv, hd=HD, out_dtype=torch.float16)
    G = n_heads // n_kv
    Q = qt.view(n, n_heads, HD).float()
    K, V = kt.view(n, n_kv, HD).float(), vt.view(n, n_kv, HD).float()
    mask = torch.arange(n, device=gpu)[None, :] > torch.arange(n, device=gpu)[:, None]
    ref = torch.empty((n, n_heads, HD), dtype=torch.float32, device=gpu)
    for h in range(n_heads):
        s = (Q[:, h] @ K[:, h // G].T) / HD ** 0.5
        s.masked_fill_(mask, float("-inf"))
        ref[:, h] = torch.softmax(s, dim=-1) @ V[:, h // G]
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    assert_close(got, ref.view(n, -1).cpu().numpy(), what="prefill hd256 4096 vs torch fp32")
    for r in (0, 31, 32, 127, 128, 4095):
        assert_close(got[r:r + 1], reference_f64(q[r:r + 1], k, v, r, n_heads, n_kv, hd=HD),
                     what=f"prefill hd256 row {r} vs f64")


def test_chunked_prefill_hd256_matches_whole_prompt(gpu):
    n, chunk, n_heads, n_kv = 768, 256, 16, 2
    q, k, v = make_inputs(72, n, n, n_heads, n_kv, hd=HD, q_dtype=np.float16)
    qt, kt, vt = to_dev(q, k, v, gpu, n_kv)
    whole = gi_attn.prefill(qt, kt, vt, 0, n_heads, n_kv, hd=HD, out_dtype=torch.float32)
    parts = []
    for c0 in range(0, n, chunk):
        say("hd256 chunk at", c0)
        parts.append(gi_attn.prefill(qt[c0:c0 + chunk], kt, vt, c0, n_heads, n_kv, hd=HD, out_dtype=torch.float32))
    torch.cuda.synchronize()
    assert np.array_equal(torch.cat(parts).cpu().numpy(), whole.cpu().numpy())


@pytest.mark.parametrize("n,pos0,exact", [(1, 99, False), (8, 300, True), (20, 0, False), (40, 17, True)])
def test_attention_operator_hd256(gpu, n, pos0, exact):
    say("operator hd256", n, pos0, exact)
    n_heads, n_kv = 16, 2
    row = n_heads * HD + 2 * n_kv * HD
    qkv = np.random.default_rng(97 + n).standard_normal((n, row), dtype=np.float32)
    _, k, v = make_inputs(98 + n, 1, pos0 + n, n_heads, n_kv, hd=HD)
    qkv_t = torch.from_numpy(qkv).to(gpu)
    _, kt, vt = to_dev(qkv[:, :1], k, v, gpu, n_kv)
    out = gi_attn.attention(qkv_t, kt, vt, pos0, n_heads, n_kv, hd=HD, exact=exact)
    torch.cuda.synchronize()
    q = np.ascontiguousarray(qkv[:, :n_heads * HD])
    split_path = n < 16 or exact
    assert_close(out.cpu().numpy(), reference_f64(q, k, v, pos0, n_heads, n_kv, hd=HD),
                 max_abs=2e-5 if split_path else 2e-3, rel_l2=2e-5 if split_path else 1e-3,
                 what="operator hd256 vs f64")


# ---------------------------------------------------------------- prefill over the int8 cache (attn_prefill_tc<256, 2>
# with KV8): integer keys times their scale on the score, f16(p * vscale * 2^10) for P V, output / 2^10 / l

PREFILL_SHAPES_256_I8 = [
    (16, 0, 8, 2, "reference"),
    (65, 0, 4, 1, "reference"),
    (127, 63, 8, 2, "head_major"),
    (129, 0, 8, 8, "reference"),
    (300, 40, 16, 2, "head_major"),
    (1000, 24, 16, 2, "reference"),
]


@pytest.mark.parametrize("n,pos0,n_heads,n_kv,layout", PREFILL_SHAPES_256_I8)
def test_prefill_hd256_i8(gpu, n, pos0, n_heads, n_kv, layout):
    say("prefill hd256 i8", n, pos0, n_heads, n_kv, layout)
    q, k, v, ks, vs = make_inputs_i8(8100 + n + pos0, n, pos0 + n, n_heads, n_kv, hd=HD)
    qt, kt, vt, kst, vst = to_dev_i8(q, k, v, ks, vs, gpu, n_kv, layout)
    out = gi_attn.prefill(qt, kt, vt, pos0, n_heads, n_kv, hd=HD, out_dtype=torch.float32, kv_layout=layout,
                          k_scale=kst, v_scale=vst)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert_close(got, O.prefill_tc_semantics_i8(q, k, v, ks, vs, pos0, n_heads, n_kv, hd=HD),
                 what="prefill hd256 i8 vs oracle (attention_prefill_tc256 with KV8)")
    assert_close(got, reference_f64_i8(q, k, v, ks, vs, pos0, n_heads, n_kv, hd=HD), what="prefill hd256 i8 vs f64")


def test_prefill_hd256_i8_4096_and_chunks(gpu):
    # a 4096-token prompt over the int8 cache: sampled rows against float64, and chunks of 1024 at their prefix
    # give the whole prompt's rows bit for bit
    n, n_heads, n_kv = 4096, 16, 2
    say("prefill hd256 i8 4096")
    q, k, v, ks, vs = make_inputs_i8(83, n, n, n_heads, n_kv, hd=HD)
    qt, kt, vt, kst, vst = to_dev_i8(q, k, v, ks, vs, gpu, n_kv)
    whole = gi_attn.prefill(qt, kt, vt, 0, n_heads, n_kv, hd=HD, k_scale=kst, v_scale=vst)
    parts = [gi_attn.prefill(qt[c0:c0 + 1024], kt, vt, c0, n_heads, n_kv, hd=HD, k_scale=kst, v_scale=vst)
             for c0 in range(0, n, 1024)]
    torch.cuda.synchronize()
    got = whole.cpu().numpy()
    for r in (0, 31, 127, 128, 2047, 4095):
        assert_close(got[r:r + 1], reference_f64_i8(q[r:r + 1], k, v, ks, vs, r, n_heads, n_kv, hd=HD),
                     what=f"prefill hd256 i8 row {r} vs f64")
    assert np.array_equal(torch.cat(parts).cpu().numpy(), got)


@pytest.mark.parametrize("n,pos0,exact", [(1, 99, False), (8, 300, True), (20, 0, False), (40, 17, True)])
def test_attention_operator_hd256_i8(gpu, n, pos0, exact):
    say("operator hd256 i8", n, pos0, exact)
    n_heads, n_kv = 16, 2
    row = n_heads * HD + 2 * n_kv * HD
    qkv = np.random.default_rng(197 + n).standard_normal((n, row), dtype=np.float32)
    _, k, v, ks, vs = make_inputs_i8(198 + n, 1, pos0 + n, n_heads, n_kv, hd=HD)
    qkv_t = torch.from_numpy(qkv).to(gpu)
    _, kt, vt, kst, vst = to_dev_i8(qkv[:, :1], k, v, ks, vs, gpu, n_kv)
    out = gi_attn.attention(qkv_t, kt, vt, pos0, n_heads, n_kv, hd=HD, exact=exact, k_scale=kst, v_scale=vst)
    torch.cuda.synchronize()
    q = np.ascontiguousarray(qkv[:, :n_heads * HD])
    assert_close(out.cpu().numpy(), reference_f64_i8(q, k, v, ks, vs, pos0, n_heads, n_kv, hd=HD),
                 *split_f64_tol("i8", HD), what="operator hd256 i8 vs f64")
