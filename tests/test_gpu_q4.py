"""Parity of the 4-bit KV cache (the reference's --kv q4, src/cuda.rs:226-256) on the gfx950 kernels, through the
C ABI: the rotated store (qk_norm_rope with KV4), the tensor-core decode over it (attention_decode_tc256 with KV4)
and, end to end, the attention of the unrotated rows.

Bar: the cache bytes and scales bit-exact against the oracle's quantiser (on the same rotated rows, and on the
same input for v rows, whose rotation is bit-identical to kv4_fwht); decode outputs within REF_ORACLE_TOL of the
oracle's restatement of attention_decode_tc256 (the same f16 roundings of Q and P) and within max-abs 2e-3 /
relative L2 1e-3 of float64 attention over the cache's f16 values.
"""
import sys

import numpy as np
import pytest
import torch

import gi_attn
import gi_oracle as O
from attn_common import REF_ORACLE_TOL, assert_close, make_inputs_q4, reference_f64_q4, split_f64_tol

F64_TOL = split_f64_tol("q4", 256)

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


def q4_dev(q, kc, vc, ks, vs, dev, n_kv, layout="reference"):
    qt = torch.from_numpy(np.ascontiguousarray(q)).to(dev)
    kt = torch.from_numpy(np.ascontiguousarray(kc)).to(dev).view(-1, n_kv, 128)
    vt = torch.from_numpy(np.ascontiguousarray(vc)).to(dev).view(-1, n_kv, 128)
    kst = torch.from_numpy(np.ascontiguousarray(ks).view(np.float16)).to(dev).view(-1, n_kv, 8)
    vst = torch.from_numpy(np.ascontiguousarray(vs).view(np.float16)).to(dev).view(-1, n_kv, 8)
    if layout == "head_major":
        kt, vt, kst, vst = (t.transpose(0, 1).contiguous() for t in (kt, vt, kst, vst))
    return qt, kt, vt, kst, vst


DECODE_SHAPES_Q4 = [
    # (n_tok, pos0, n_heads, n_kv): spans inside one 16-key tile and at tile / slice edges, both kernel variants
    # (up to 16 pairs per kv head: one column block per workgroup; above: two column blocks per wave), G = 3
    (1, 0, 16, 2),
    (1, 15, 16, 2),
    (1, 64, 16, 2),
    (1, 4095, 16, 2),
    (2, 300, 8, 2),
    (3, 77, 12, 4),
    (8, 2000, 16, 2),
    (15, 513, 16, 2),
    (1, 40000, 16, 2),
    (8, 249, 16, 2),  # token 0's span ends before the last slice: its partial there is empty (m = -inf) and the merge skips it
    (2, 63, 16, 2),    # the same with 4 pairs: token 0 sees all of slice 0 and none of slice 1
]


@pytest.mark.parametrize("n_tok,pos0,n_heads,n_kv", DECODE_SHAPES_Q4)
def test_decode_q4(gpu, n_tok, pos0, n_heads, n_kv):
    say("decode q4", n_tok, pos0, n_heads, n_kv)
    q, kc, vc, ks, vs = make_inputs_q4(500 + pos0 + n_tok, n_tok, pos0 + n_tok, n_heads, n_kv)
    t = q4_dev(q, kc, vc, ks, vs, gpu, n_kv)
    out = gi_attn.decode_q4(*t, pos0, n_heads, n_kv)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert_close(got, O.decode_tc256_q4(q, kc, vc, ks, vs, pos0, n_heads, n_kv), *REF_ORACLE_TOL,
                 what="q4 decode vs oracle")
    assert_close(got, reference_f64_q4(q, kc, vc, ks, vs, pos0, n_heads, n_kv), *F64_TOL, what="q4 decode vs f64")


@pytest.mark.parametrize("n_tok", [1, 8])
def test_decode_q4_head_major_and_device_position(gpu, n_tok):
    # the head-major layout, and a device position (graph replay's posp) with the launch sized for ctx_cap
    n_heads, n_kv, cap, pos0 = 16, 2, 3000, 2500
    say("decode q4 head-major posp", n_tok)
    q, kc, vc, ks, vs = make_inputs_q4(77 + n_tok, n_tok, cap, n_heads, n_kv)
    t = q4_dev(q, kc, vc, ks, vs, gpu, n_kv, layout="head_major")
    posp = torch.full((1,), pos0, dtype=torch.int32, device=gpu)
    out = gi_attn.decode_q4(*t, 0, n_heads, n_kv, posp=posp, ctx_cap=cap, kv_layout="head_major")
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert_close(got, O.decode_tc256_q4(q, kc, vc, ks, vs, pos0, n_heads, n_kv), *REF_ORACLE_TOL,
                 what="q4 decode head-major posp vs oracle")
    assert_close(got, reference_f64_q4(q, kc, vc, ks, vs, pos0, n_heads, n_kv), *F64_TOL,
                 what="q4 decode head-major posp vs f64")


@pytest.mark.parametrize("n_tok", [1, 8])
def test_decode_q4_graph_replay(gpu, n_tok):
    # a device position, the launch captured once and replayed at several positions with eager work between the
    # replays (one column block per workgroup at 1 token, two column blocks per wave at 8)
    n_heads, n_kv, cap = 16, 2, 2500
    q, kc, vc, ks, vs = make_inputs_q4(96 + n_tok, n_tok, cap, n_heads, n_kv)
    t = q4_dev(q, kc, vc, ks, vs, gpu, n_kv)
    ws = gi_attn.new_workspace(cap, n_tok, n_heads, n_kv, hd=256, device=gpu)
    posp = torch.zeros(1, dtype=torch.int32, device=gpu)
    out = torch.zeros((n_tok, n_heads * 256), dtype=torch.float32, device=gpu)
    kw = dict(out=out, workspace=ws, posp=posp, ctx_cap=cap)
    gi_attn.decode_q4(*t, 0, n_heads, n_kv, **kw)  # warm-up
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        gi_attn.decode_q4(*t, 0, n_heads, n_kv, **kw)
    for pos in (cap - n_tok, 17, 1000, 0):
        say("decode q4 graph replay", n_tok, pos)
        posp.fill_(pos)
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        assert_close(got, O.decode_tc256_q4(q, kc, vc, ks, vs, pos, n_heads, n_kv), *REF_ORACLE_TOL,
                     what=f"q4 replay at {pos} vs oracle")
        assert_close(got, reference_f64_q4(q, kc, vc, ks, vs, pos, n_heads, n_kv), *F64_TOL,
                     what=f"q4 replay at {pos} vs f64")


@pytest.mark.parametrize("n,H,K,ctx,pos0", [(7, 8, 2, 40, 11), (1, 16, 2, 5000, 4999), (200, 4, 1, 260, 50),
                                            (33, 32, 4, 100, 60)])
def test_rope_q4_store_is_bit_exact(gpu, n, H, K, ctx, pos0):
    # q/k heads: RMSNorm + RoPE + rotation, against the oracle within f32 rounding (sincos and pow differ by
    # ulps, and a rotation angle of a few thousand radians moves by ~1e-4 at large positions); the k cache: the
    # oracle's quantiser of the kernel's own rotated k rows, bit for bit; the v cache: rotation and quantiser of
    # the same input, bit for bit
    rng = np.random.default_rng(21 + n)
    qkv = rng.standard_normal((n, (H + 2 * K) * 256)).astype(np.float32)
    qn = rng.uniform(0.5, 1.5, 256).astype(np.float32)
    kn = rng.uniform(0.5, 1.5, 256).astype(np.float32)
    z8 = np.zeros((ctx, K * 128), np.uint8)
    z16 = np.zeros((ctx, K * 8), np.uint16)
    want, wkc, wvc, wks, wvs = O.qk_norm_rope_q4(qkv, z8, z8, z16, z16, pos0, H, K, qn=qn, kn=kn)
    say("rope q4 store", n, H, K, ctx, pos0)
    x = torch.from_numpy(qkv).to(gpu)
    kc = torch.zeros((ctx, K, 128), dtype=torch.uint8, device=gpu)
    vc = torch.zeros_like(kc)
    ks = torch.zeros((ctx, K, 8), dtype=torch.float16, device=gpu)
    vs = torch.zeros_like(ks)
    gi_attn.qk_norm_rope_q4(x, kc, vc, ks, vs, pos0, H, K, qn=torch.from_numpy(qn).to(gpu),
                            kn=torch.from_numpy(kn).to(gpu))
    torch.cuda.synchronize()
    got = x.cpu().numpy()
    np.testing.assert_allclose(got, want, rtol=0, atol=2e-5 if pos0 + n < 100 else 2e-3)
    krot = got[:, H * 256:(H + K) * 256].reshape(n * K, 256)
    kq, ksq = O.kv4_quant(krot)
    np.testing.assert_array_equal(kc.cpu().numpy()[pos0:pos0 + n].reshape(n * K, 128), kq)
    np.testing.assert_array_equal(ks.cpu().numpy()[pos0:pos0 + n].reshape(n * K, 8).view(np.uint16), ksq)
    np.testing.assert_array_equal(vc.cpu().numpy().reshape(ctx, -1), wvc)
    np.testing.assert_array_equal(vs.cpu().numpy().reshape(ctx, -1).view(np.uint16), wvs)
    assert not kc[:pos0].any() and not kc[pos0 + n:].any()


def test_rope_q4_rotation_is_bit_identical(gpu):
    # without norm and RoPE (rope_dim 0) the q and k heads are only rotated: the kernel's transform equals
    # kv4_fwht bit for bit, on rows with values of every magnitude
    n, H, K, ctx = 5, 4, 2, 8
    rng = np.random.default_rng(22)
    qkv = (rng.standard_normal((n, (H + 2 * K) * 256)) * np.exp(rng.uniform(-8, 8, (n, (H + 2 * K) * 256))))
    qkv = qkv.astype(np.float32)
    say("rope q4 rotation")
    x = torch.from_numpy(qkv).to(gpu)
    kc = torch.zeros((ctx, K, 128), dtype=torch.uint8, device=gpu)
    vc = torch.zeros_like(kc)
    ks = torch.zeros((ctx, K, 8), dtype=torch.float16, device=gpu)
    vs = torch.zeros_like(ks)
    gi_attn.qk_norm_rope_q4(x, kc, vc, ks, vs, 0, H, K, rope_dim=0)
    torch.cuda.synchronize()
    qk = qkv[:, :(H + K) * 256].reshape(-1, 256)
    np.testing.assert_array_equal(x.cpu().numpy()[:, :(H + K) * 256], O.kv4_fwht(qk).reshape(n, -1))
    vq, vsq = O.kv4_quant(O.kv4_fwht(qkv[:, (H + K) * 256:].reshape(-1, 256)))
    np.testing.assert_array_equal(vc.cpu().numpy()[:n].reshape(n * K, 128), vq)
    np.testing.assert_array_equal(vs.cpu().numpy()[:n].reshape(n * K, 8).view(np.uint16), vsq)


def test_q4_layer_end_to_end(gpu):
    # a prompt's rows through the rotated store, then a decode step: the output, rotated back on the host with
    # kv4_fwht, is the attention of the unrotated rows to within the 4-bit rounding, and equals the oracle's
    # KV4 decode over the kernel's own cache at the parity bar
    H, K, n, ctx = 16, 2, 600, 1024
    rng = np.random.default_rng(23)
    qkv = rng.standard_normal((n, (H + 2 * K) * 256)).astype(np.float32)
    x = torch.from_numpy(qkv).to(gpu)
    kc = torch.zeros((ctx, K, 128), dtype=torch.uint8, device=gpu)
    vc = torch.zeros_like(kc)
    ks = torch.zeros((ctx, K, 8), dtype=torch.float16, device=gpu)
    vs = torch.zeros_like(ks)
    say("q4 end to end")
    gi_attn.qk_norm_rope_q4(x, kc, vc, ks, vs, 0, H, K, rope_dim=0)
    qrot = x[n - 1:, :H * 256].contiguous()
    out = gi_attn.decode_q4(qrot, kc, vc, ks, vs, n - 1, H, K)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    c = [t.cpu().numpy().reshape(ctx, -1) for t in (kc, vc, ks, vs)]
    c[2], c[3] = c[2].view(np.uint16), c[3].view(np.uint16)
    assert_close(got, O.decode_tc256_q4(qrot.cpu().numpy(), *c, n - 1, H, K), *REF_ORACLE_TOL, what="q4 e2e vs oracle")
    back = O.kv4_fwht(got.reshape(-1, 256)).reshape(1, -1)
    from attn_common import _reference_f64_values
    exact = _reference_f64_values(qkv[n - 1:, :H * 256], qkv[:, H * 256:(H + K) * 256], qkv[:, (H + K) * 256:],
                                  n - 1, H, K, 256)
    assert np.abs(back - exact).max() < 0.05


PREFILL_SHAPES_Q4 = [
    # (n, pos0, n_heads, n_kv, q dtype, layout): one tile, diagonal and tile edges (64 keys, 128 query rows per
    # workgroup), chunks at a prefix, both layouts
    (16, 0, 8, 2, np.float32, "reference"),
    (65, 0, 4, 1, np.float16, "reference"),
    (127, 63, 8, 2, np.float32, "head_major"),
    (129, 0, 8, 8, np.float32, "reference"),
    (300, 40, 16, 2, np.float16, "head_major"),
    (1000, 24, 16, 2, np.float32, "reference"),
]


@pytest.mark.parametrize("n,pos0,n_heads,n_kv,qd,layout", PREFILL_SHAPES_Q4)
def test_prefill_q4(gpu, n, pos0, n_heads, n_kv, qd, layout):
    say("prefill q4", n, pos0, n_heads, n_kv, qd.__name__, layout)
    q, kc, vc, ks, vs = make_inputs_q4(900 + n + pos0, n, pos0 + n, n_heads, n_kv)
    q = q.astype(qd)
    t = q4_dev(q, kc, vc, ks, vs, gpu, n_kv, layout)
    out = gi_attn.prefill_q4(*t, pos0, n_heads, n_kv, out_dtype=torch.float32, kv_layout=layout)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    q32 = q.astype(np.float32)
    assert_close(got, O.prefill_tc256_q4(q32, kc, vc, ks, vs, pos0, n_heads, n_kv),
                 what="prefill q4 vs oracle (attention_prefill_tc256 with KV4)")
    assert_close(got, reference_f64_q4(q32, kc, vc, ks, vs, pos0, n_heads, n_kv), what="prefill q4 vs f64")


def test_prefill_q4_4096_and_chunks(gpu):
    n, n_heads, n_kv = 4096, 16, 2
    say("prefill q4 4096")
    q, kc, vc, ks, vs = make_inputs_q4(91, n, n, n_heads, n_kv)
    t = q4_dev(q, kc, vc, ks, vs, gpu, n_kv)
    whole = gi_attn.prefill_q4(*t, 0, n_heads, n_kv)
    parts = [gi_attn.prefill_q4(t[0][c0:c0 + 1024], *t[1:], c0, n_heads, n_kv) for c0 in range(0, n, 1024)]
    torch.cuda.synchronize()
    got = whole.cpu().numpy()
    for r in (0, 31, 127, 128, 2047, 4095):
        assert_close(got[r:r + 1], reference_f64_q4(q[r:r + 1], kc, vc, ks, vs, r, n_heads, n_kv),
                     what=f"prefill q4 row {r} vs f64")
    assert np.array_equal(torch.cat(parts).cpu().numpy(), got)


def test_hadamard_rows_bit_exact(gpu):
    # hadamard_rows with block 256: every segment of every row equals kv4_fwht's bits (also with a row stride
    # wider than the rows)
    rng = np.random.default_rng(31)
    x = (rng.standard_normal((37, 16 * 256)) * np.exp(rng.uniform(-10, 10, (37, 16 * 256)))).astype(np.float32)
    say("hadamard rows")
    big = torch.zeros((37, 16 * 256 + 64), dtype=torch.float32, device=gpu)
    big[:, :16 * 256] = torch.from_numpy(x).to(gpu)
    view = big[:, :16 * 256]
    gi_attn.hadamard_rows(view)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(view.cpu().numpy(), O.kv4_fwht(x.reshape(-1, 256)).reshape(37, -1))
    assert not big[:, 16 * 256:].any()


@pytest.mark.parametrize("n,pos0,exact", [(1, 99, False), (8, 300, True), (20, 0, False), (40, 17, True)])
def test_attention_operator_q4(gpu, n, pos0, exact):
    # GpuModel::attention over the 4-bit cache: prefill from 16 tokens unless exact, else the split decode path;
    # then hadamard_rows turns the output back, and it is the attention of the unrotated queries over the
    # unrotated cache rows (the cache's f16 values rotated back in float64)
    say("operator q4", n, pos0, exact)
    n_heads, n_kv = 16, 2
    row = (n_heads + 2 * n_kv) * 256
    qkv = np.random.default_rng(297 + n).standard_normal((n, row), dtype=np.float32)
    _, kc, vc, ks, vs = make_inputs_q4(298 + n, 1, pos0 + n, n_heads, n_kv)
    qkv_t = torch.from_numpy(qkv).to(gpu)
    _, kt, vt, kst, vst = q4_dev(qkv[:, :1], kc, vc, ks, vs, gpu, n_kv)
    out = gi_attn.attention_q4(qkv_t, kt, vt, kst, vst, pos0, n_heads, n_kv, exact=exact)
    gi_attn.hadamard_rows(out)
    torch.cuda.synchronize()
    q = np.ascontiguousarray(qkv[:, :n_heads * 256])
    rot = reference_f64_q4(q, kc, vc, ks, vs, pos0, n_heads, n_kv)
    want = (rot.reshape(-1, 256) @ _h256()).reshape(rot.shape)
    assert_close(out.cpu().numpy(), want, *F64_TOL, what="operator q4 (rotated back) vs f64")


def _h256():
    i = np.arange(256)
    bits = np.vectorize(lambda x: bin(x).count("1"))(i[:, None] & i[None, :])
    return np.where(bits % 2 == 0, 1.0, -1.0) / 16.0
