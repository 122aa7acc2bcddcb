"""Parity of head size 64 on the gfx950 kernels, through the C ABI: the reference's attention_partial_gqa at a head
size of 64 (any multiple of 32, src/cuda.rs:1684-1865, 8419-8422) and attention_prefill_tc64 (attn_prefill_tc<64>,
src/cuda.rs:2620, dispatched at src/cuda.rs:8452-8456), over the f16 and the int8 cache. SmolLM2-135M, the
reference's documented test model (docs/building.md:58), has 9 query heads, 3 kv heads and 64-wide heads.

Bar: decode within 2e-5 of float64 (f32 precision, as at head size 128) and within the north star's bar of the
oracle's Model::attention (src/model.rs:1320-1409); prefill within the bar of the oracle's attn_prefill_tc<64>
restatement and of float64 (it rounds Q and P to f16 as the reference does)."""
import sys

import numpy as np
import pytest
import torch

import gi_attn
import gi_oracle as O
from attn_common import (SPLIT_F64_TOL, assert_close, make_inputs, make_inputs_i8, reference_f64, reference_f64_i8)

pytestmark = pytest.mark.gpu
HD = 64


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


def to_dev_i8(q, k, v, ks, vs, dev, n_kv, layout="reference"):
    if layout == "head_major":
        k = np.ascontiguousarray(k.reshape(k.shape[0], n_kv, HD).transpose(1, 0, 2))
        v = np.ascontiguousarray(v.reshape(v.shape[0], n_kv, HD).transpose(1, 0, 2))
        ks, vs = np.ascontiguousarray(ks.T), np.ascontiguousarray(vs.T)
    return [torch.from_numpy(np.ascontiguousarray(x)).to(dev) for x in (q, k, v, ks, vs)]


DECODE_SHAPES_64 = [
    # (n_tok, pos0, n_heads, n_kv): every kernel variant (up to 8 (token, head) pairs per kv head: hi/lo columns;
    # up to 16: one pair per column; above: two column blocks per wave, 32 pairs per workgroup), spans inside one
    # tile, at tile and slice edges, and long; SmolLM2's 9/3 heads (G = 3)
    (1, 0, 9, 3),
    (1, 31, 9, 3),
    (1, 127, 9, 3),
    (1, 4095, 9, 3),
    (2, 300, 9, 3),     # 6 pairs
    (5, 77, 9, 3),      # 15 pairs: one column block
    (8, 2000, 9, 3),    # 24 pairs: two column blocks
    (15, 513, 9, 3),    # 45 pairs: two pair groups
    (1, 40000, 32, 8),  # G = 4, long context
    (3, 60, 16, 1),     # G = 16: 48 pairs on one kv head
    (1, 1000, 32, 2),   # G = 16, one token
    (16, 1000, 4, 4),   # G = 1
    (8, 249, 16, 4),  # token 0's span ends before the last slice: its partial there is empty (m = -inf) and the merge skips it
]


@pytest.mark.parametrize("n_tok,pos0,n_heads,n_kv", DECODE_SHAPES_64)
def test_decode_hd64(gpu, n_tok, pos0, n_heads, n_kv):
    say("decode hd64", n_tok, pos0, n_heads, n_kv)
    q, k, v = make_inputs(9000 + pos0 + n_tok, n_tok, pos0 + n_tok, n_heads, n_kv, hd=HD)
    qt, kt, vt = to_dev(q, k, v, gpu, n_kv)
    out = gi_attn.decode(qt, kt, vt, pos0, n_heads, n_kv, hd=HD)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert_close(got, O.attention(q, k, v, pos0, n_heads, n_kv, hd=HD), what="decode hd64 vs oracle (Model::attention)")
    assert_close(got, reference_f64(q, k, v, pos0, n_heads, n_kv, hd=HD), *SPLIT_F64_TOL, what="decode hd64 vs f64")


@pytest.mark.parametrize("n_tok,pos0,n_heads,n_kv", DECODE_SHAPES_64)
def test_decode_hd64_i8(gpu, n_tok, pos0, n_heads, n_kv):
    say("decode hd64 i8", n_tok, pos0, n_heads, n_kv)
    q, k, v, ks, vs = make_inputs_i8(9100 + pos0 + n_tok, n_tok, pos0 + n_tok, n_heads, n_kv, hd=HD)
    qt, kt, vt, kst, vst = to_dev_i8(q, k, v, ks, vs, gpu, n_kv)
    out = gi_attn.decode(qt, kt, vt, pos0, n_heads, n_kv, hd=HD, k_scale=kst, v_scale=vst)
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), reference_f64_i8(q, k, v, ks, vs, pos0, n_heads, n_kv, hd=HD), *SPLIT_F64_TOL,
                 what="decode hd64 i8 vs f64")


@pytest.mark.parametrize("n_tok,i8", [(1, False), (8, False), (1, True), (8, True)])
def test_decode_hd64_head_major_graph_replay(gpu, n_tok, i8):
    # the head-major layout and a device position, the launch captured once and replayed at several positions with
    # eager work between the replays
    n_heads, n_kv, cap = 9, 3, 2500
    if i8:
        q, k, v, ks, vs = make_inputs_i8(97 + n_tok, n_tok, cap, n_heads, n_kv, hd=HD)
        qt, kt, vt, kst, vst = to_dev_i8(q, k, v, ks, vs, gpu, n_kv, "head_major")
        sc = dict(k_scale=kst, v_scale=vst)
    else:
        q, k, v = make_inputs(98 + n_tok, n_tok, cap, n_heads, n_kv, hd=HD)
        qt, kt, vt = to_dev(q, k, v, gpu, n_kv, "head_major")
        sc = {}
    ws = gi_attn.new_workspace(cap, n_tok, n_heads, n_kv, hd=HD, device=gpu)
    posp = torch.zeros(1, dtype=torch.int32, device=gpu)
    out = torch.zeros((n_tok, n_heads * HD), dtype=torch.float32, device=gpu)
    kw = dict(hd=HD, out=out, workspace=ws, posp=posp, ctx_cap=cap, kv_layout="head_major", **sc)
    gi_attn.decode(qt, kt, vt, 0, n_heads, n_kv, **kw)  # warm-up
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        gi_attn.decode(qt, kt, vt, 0, n_heads, n_kv, **kw)
    for pos in (cap - n_tok, 31, 1000, 0):
        say("decode hd64 graph replay", n_tok, i8, pos)
        posp.fill_(pos)
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        want = (reference_f64_i8(q, k, v, ks, vs, pos, n_heads, n_kv, hd=HD) if i8
                else reference_f64(q, k, v, pos, n_heads, n_kv, hd=HD))
        assert_close(out.cpu().numpy(), want, *SPLIT_F64_TOL, what=f"hd64 replay at {pos}")


# ---------------------------------------------------------------- prefill (attention_prefill_tc64)

PREFILL_SHAPES_64 = [
    # (n, pos0, n_heads, n_kv, q dtype, out dtype, layout): one tile, diagonal and tile edges (64 keys, 256 query
    # rows per workgroup), chunks at a prefix, both layouts
    (16, 0, 9, 3, np.float16, torch.float32, "reference"),
    (33, 0, 4, 1, np.float32, torch.float32, "reference"),
    (65, 0, 9, 3, np.float16, torch.float32, "head_major"),
    (255, 1, 8, 2, np.float16, torch.float16, "reference"),
    (257, 0, 9, 3, np.float32, torch.float32, "reference"),
    (300, 40, 16, 2, np.float16, torch.float32, "head_major"),
    (70, 130, 8, 8, np.float16, torch.float32, "reference"),
    (1000, 24, 9, 3, np.float16, torch.float32, "reference"),
]


@pytest.mark.parametrize("n,pos0,n_heads,n_kv,qd,od,layout", PREFILL_SHAPES_64)
def test_prefill_hd64(gpu, n, pos0, n_heads, n_kv, qd, od, layout):
    say("prefill hd64", n, pos0, n_heads, n_kv, qd.__name__, od, layout)
    q, k, v = make_inputs(9200 + n + pos0, n, pos0 + n, n_heads, n_kv, hd=HD, q_dtype=qd)
    qt, kt, vt = to_dev(q, k, v, gpu, n_kv, layout)
    out = gi_attn.prefill(qt, kt, vt, pos0, n_heads, n_kv, hd=HD, out_dtype=od, kv_layout=layout)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    q32 = q.astype(np.float32)
    assert_close(got, O.prefill_tc_semantics(q32, k, v, pos0, n_heads, n_kv, hd=HD),
                 what="prefill hd64 vs oracle (attention_prefill_tc64 semantics)")
    assert_close(got, reference_f64(q32, k, v, pos0, n_heads, n_kv, hd=HD), what="prefill hd64 vs f64")


def test_prefill_hd64_4096_and_chunks(gpu):
    # a 4096-token prompt at SmolLM2's shape: the whole output against a torch fp32 reference on the GPU, sampled rows
    # against float64, and chunks of 1024 at their prefix equal to the whole prompt's rows bit for bit
    n, n_heads, n_kv = 4096, 9, 3
    say("prefill hd64 4096 9q/3kv")
    q, k, v = make_inputs(73, n, n, n_heads, n_kv, hd=HD, q_dtype=np.float16)
    qt, kt, vt = to_dev(q, k, v, gpu, n_kv)
    out = gi_attn.prefill(qt, kt, vt, 0, n_heads, n_kv, hd=HD, out_dtype=torch.float32)
    parts = [gi_attn.prefill(qt[c0:c0 + 1024], kt, vt, c0, n_heads, n_kv, hd=HD, out_dtype=torch.float32)
             for c0 in range(0, n, 1024)]
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
    got = out.cpu().numpy()
    assert_close(got, ref.view(n, -1).cpu().numpy(), what="prefill hd64 4096 vs torch fp32")
    for r in (0, 31, 255, 256, 4095):
        assert_close(got[r:r + 1], reference_f64(q[r:r + 1], k, v, r, n_heads, n_kv, hd=HD),
                     what=f"prefill hd64 row {r} vs f64")
    assert np.array_equal(torch.cat(parts).cpu().numpy(), got)


PREFILL_SHAPES_64_I8 = [
    (16, 0, 9, 3, "reference"),
    (65, 0, 4, 1, "reference"),
    (255, 1, 9, 3, "head_major"),
    (257, 0, 8, 8, "reference"),
    (300, 40, 16, 2, "head_major"),
    (1000, 24, 9, 3, "reference"),
]


@pytest.mark.parametrize("n,pos0,n_heads,n_kv,layout", PREFILL_SHAPES_64_I8)
def test_prefill_hd64_i8(gpu, n, pos0, n_heads, n_kv, layout):
    say("prefill hd64 i8", n, pos0, n_heads, n_kv, layout)
    q, k, v, ks, vs = make_inputs_i8(9300 + n + pos0, n, pos0 + n, n_heads, n_kv, hd=HD)
    qt, kt, vt, kst, vst = to_dev_i8(q, k, v, ks, vs, gpu, n_kv, layout)
    out = gi_attn.prefill(qt, kt, vt, pos0, n_heads, n_kv, hd=HD, out_dtype=torch.float32, kv_layout=layout,
                          k_scale=kst, v_scale=vst)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert_close(got, O.prefill_tc_semantics_i8(q, k, v, ks, vs, pos0, n_heads, n_kv, hd=HD),
                 what="prefill hd64 i8 vs oracle (attention_prefill_tc64 with KV8)")
    assert_close(got, reference_f64_i8(q, k, v, ks, vs, pos0, n_heads, n_kv, hd=HD), what="prefill hd64 i8 vs f64")


# ---------------------------------------------------------------- the operator (GpuModel::attention)

@pytest.mark.parametrize("n,pos0,exact,i8", [(1, 99, False, False), (8, 300, True, False), (20, 0, False, False),
                                             (40, 17, True, False), (1, 99, False, True), (20, 0, False, True),
                                             (40, 17, True, True)])
def test_attention_operator_hd64(gpu, n, pos0, exact, i8):
    # SmolLM2's 9/3 heads over the reference's qkv rows: prefill from 16 tokens unless exact, else the split path
    say("operator hd64", n, pos0, exact, i8)
    n_heads, n_kv = 9, 3
    row = (n_heads + 2 * n_kv) * HD
    qkv = np.random.default_rng(397 + n).standard_normal((n, row), dtype=np.float32)
    qkv_t = torch.from_numpy(qkv).to(gpu)
    q = np.ascontiguousarray(qkv[:, :n_heads * HD])
    if i8:
        _, k, v, ks, vs = make_inputs_i8(398 + n, 1, pos0 + n, n_heads, n_kv, hd=HD)
        _, kt, vt, kst, vst = to_dev_i8(qkv[:, :1], k, v, ks, vs, gpu, n_kv)
        out = gi_attn.attention(qkv_t, kt, vt, pos0, n_heads, n_kv, hd=HD, exact=exact, k_scale=kst, v_scale=vst)
        want = reference_f64_i8(q, k, v, ks, vs, pos0, n_heads, n_kv, hd=HD)
    else:
        _, k, v = make_inputs(398 + n, 1, pos0 + n, n_heads, n_kv, hd=HD)
        _, kt, vt = to_dev(qkv[:, :1], k, v, gpu, n_kv)
        out = gi_attn.attention(qkv_t, kt, vt, pos0, n_heads, n_kv, hd=HD, exact=exact)
        want = reference_f64(q, k, v, pos0, n_heads, n_kv, hd=HD)
    torch.cuda.synchronize()
    split_path = n < 16 or exact
    assert_close(out.cpu().numpy(), want, *(SPLIT_F64_TOL if split_path else (2e-3, 1e-3)),
                 what="operator hd64 vs f64")
