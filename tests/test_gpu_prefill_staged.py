"""The pre-widened prefill over the int8 and 4-bit caches (gi_kv_widen, then the prefill kernels that stage the
widened tiles by LDS-DMA: gi_attn_prefill_i8_ws / gi_attn_prefill_q4_ws, and the operators' prefill batches) against
the kernels that widen each tile as they stage it (gi_attn_prefill_i8 / gi_attn_prefill_q4). Both feed the same f16
values and scales to the same MFMA and softmax code, so the outputs must agree bit for bit; the oracle checks of the
int8 and 4-bit prefill (test_gpu_int8.py, test_gpu_hd256.py, test_gpu_q4.py, test_gpu_hd64.py) run the widened path,
which is the default. Semantics: attention_prefill_tc64/128/256 with KV8 (src/cuda.rs:2466-2498, 2548-2605) and
with KV4 (src/cuda.rs:2495-2514)."""
import sys

import numpy as np
import pytest
import torch

import gi_attn
from attn_common import make_inputs_i8, make_inputs_q4

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


def _i8_tensors(seed, n, pos0, n_heads, n_kv, hd, layout, dev):
    q, k, v, ks, vs = make_inputs_i8(seed, n, pos0 + n, n_heads, n_kv, hd=hd)
    kd = [np.ascontiguousarray(x) for x in (k, v, ks, vs)]
    if layout == "head_major":
        kd = [np.ascontiguousarray(x.reshape(x.shape[0], n_kv, hd).transpose(1, 0, 2)) for x in kd[:2]] + \
             [np.ascontiguousarray(x.T) for x in kd[2:]]
    return torch.from_numpy(q).to(dev), [torch.from_numpy(x).to(dev) for x in kd]


I8_SHAPES = [
    # (n, pos0, n_heads, n_kv, hd, layout, q dtype, out dtype): one tile, ragged tiles, chunks at a prefix, GQA
    (16, 0, 8, 2, 128, "reference", torch.float32, torch.float32),
    (300, 0, 32, 8, 128, "head_major", torch.float16, torch.float16),
    (257, 1000, 16, 4, 128, "reference", torch.float32, torch.float32),
    (64, 4033, 8, 1, 128, "head_major", torch.float32, torch.float16),
    (100, 0, 9, 3, 64, "reference", torch.float32, torch.float32),
    (513, 77, 32, 8, 64, "head_major", torch.float16, torch.float32),
    (40, 0, 4, 1, 256, "reference", torch.float32, torch.float32),
    (200, 300, 16, 2, 256, "head_major", torch.float16, torch.float16),
]


@pytest.mark.parametrize("n,pos0,n_heads,n_kv,hd,layout,qd,od", I8_SHAPES)
def test_prefill_i8_widened_matches_tile_widening_bit_for_bit(gpu, n, pos0, n_heads, n_kv, hd, layout, qd, od):
    say("prefill i8 staged", n, pos0, n_heads, n_kv, hd, layout, qd, od)
    q, (k, v, ks, vs) = _i8_tensors(6100 + n + pos0 + hd, n, pos0, n_heads, n_kv, hd, layout, gpu)
    q = q.to(qd)
    kw = dict(hd=hd, out_dtype=od, kv_layout=layout, k_scale=ks, v_scale=vs)
    a = gi_attn.prefill(q, k, v, pos0, n_heads, n_kv, staged=True, **kw)
    b = gi_attn.prefill(q, k, v, pos0, n_heads, n_kv, staged=False, **kw)
    torch.cuda.synchronize()
    assert torch.isfinite(a.float()).all()
    assert torch.equal(a, b), f"max diff {(a.float() - b.float()).abs().max().item()}"


@pytest.mark.parametrize("n,pos0,layout", [(16, 0, "reference"), (150, 0, "head_major"), (130, 2100, "reference")])
def test_prefill_q4_widened_matches_tile_widening_bit_for_bit(gpu, n, pos0, layout):
    say("prefill q4 staged", n, pos0, layout)
    n_heads, n_kv = 16, 2
    q, kc, vc, ks, vs = make_inputs_q4(6200 + n + pos0, n, pos0 + n, n_heads, n_kv)
    t = [np.ascontiguousarray(x) for x in (kc, vc)]
    s = [np.ascontiguousarray(x) for x in (ks, vs)]
    if layout == "head_major":
        t = [np.ascontiguousarray(x.reshape(-1, n_kv, 128).transpose(1, 0, 2)) for x in t]
        s = [np.ascontiguousarray(x.reshape(-1, n_kv, 8).transpose(1, 0, 2)) for x in s]
    else:
        t = [x.reshape(-1, n_kv, 128) for x in t]
        s = [x.reshape(-1, n_kv, 8) for x in s]
    kt, vt = (torch.from_numpy(x).to(gpu) for x in t)
    kst, vst = (torch.from_numpy(x.view(np.float16)).to(gpu) for x in s)
    qt = torch.from_numpy(q).to(gpu)
    a = gi_attn.prefill_q4(qt, kt, vt, kst, vst, pos0, n_heads, n_kv, out_dtype=torch.float32, kv_layout=layout,
                           staged=True)
    b = gi_attn.prefill_q4(qt, kt, vt, kst, vst, pos0, n_heads, n_kv, out_dtype=torch.float32, kv_layout=layout,
                           staged=False)
    torch.cuda.synchronize()
    assert torch.isfinite(a).all()
    assert torch.equal(a, b), f"max diff {(a - b).abs().max().item()}"


@pytest.mark.parametrize("hd", [64, 128, 256])
def test_operator_i8_prefill_batch_takes_either_staging(gpu, hd):
    # the operator's prefill batch: widened when its workspace holds the widened keys, else tile by tile; the same
    say("operator i8 staging", hd)
    n, pos0, n_heads, n_kv = 48, 500, (16 if hd == 256 else 8), 2
    _, k, v, ks, vs = make_inputs_i8(6300 + hd, 1, pos0 + n, n_heads, n_kv, hd=hd)
    qkv = torch.from_numpy(np.random.default_rng(6301).standard_normal((n, (n_heads + 2 * n_kv) * hd),
                                                                        dtype=np.float32)).to(gpu)
    t = [torch.from_numpy(x).to(gpu) for x in (k, v, ks, vs)]
    kc, vc = t[0].view(-1, n_kv, hd), t[1].view(-1, n_kv, hd)
    a = gi_attn.attention(qkv, kc, vc, pos0, n_heads, n_kv, hd=hd, k_scale=t[2], v_scale=t[3])
    small = torch.empty(256, dtype=torch.uint8, device=gpu)  # too small for the widened keys: tile widening
    b = gi_attn.attention(qkv, kc, vc, pos0, n_heads, n_kv, hd=hd, k_scale=t[2], v_scale=t[3], workspace=small)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def test_prefill_workspace_is_checked(gpu):
    n, pos0, n_heads, n_kv, hd = 32, 0, 8, 2, 128
    q, (k, v, ks, vs) = _i8_tensors(6400, n, pos0, n_heads, n_kv, hd, "reference", gpu)
    need = gi_attn.load_library().gi_attn_prefill_workspace_bytes(pos0 + n, n_kv, hd, 1)
    assert need > 0
    assert gi_attn.load_library().gi_attn_prefill_workspace_bytes(pos0 + n, n_kv, 96, 1) == 0  # the f32 kernels
    assert gi_attn.load_library().gi_attn_prefill_workspace_bytes(pos0 + n, n_kv, 128, 2) == 0  # 4-bit: hd 256 only
    kw = dict(hd=hd, k_scale=ks, v_scale=vs, staged=True)
    with pytest.raises(gi_attn.GiAttnError, match="workspace holds"):
        gi_attn.prefill(q, k, v, pos0, n_heads, n_kv, workspace=torch.empty(need - 256, dtype=torch.uint8,
                                                                             device=gpu), **kw)
    big = torch.empty(need + 256, dtype=torch.uint8, device=gpu)
    with pytest.raises(gi_attn.GiAttnError, match="256-byte aligned"):
        gi_attn.prefill(q, k, v, pos0, n_heads, n_kv, workspace=big[16:], **kw)
    # a workspace reused for a second, shorter call: the result does not depend on what the first left there
    first = gi_attn.prefill(q, k, v, pos0, n_heads, n_kv, workspace=big, **kw)
    q2 = q[:20].contiguous()
    second = gi_attn.prefill(q2, k, v, pos0, n_heads, n_kv, workspace=big, **kw)
    ref2 = gi_attn.prefill(q2, k, v, pos0, n_heads, n_kv, hd=hd, k_scale=ks, v_scale=vs, staged=False)
    torch.cuda.synchronize()
    assert torch.equal(second, ref2) and torch.isfinite(first).all()


def test_widened_prefill_graph_replay(gpu):
    # the widening launch and the prefill captured together, replayed with new queries and eager work between the
    # replays; every replay against the eager result
    n, pos0, n_heads, n_kv, hd = 96, 200, 8, 2, 128
    q, (k, v, ks, vs) = _i8_tensors(6500, n, pos0, n_heads, n_kv, hd, "reference", gpu)
    ws = gi_attn.prefill_workspace(pos0 + n, n_kv, hd, 1, gpu)
    out = torch.empty((n, n_heads * hd), dtype=torch.float32, device=gpu)
    kw = dict(hd=hd, k_scale=ks, v_scale=vs, workspace=ws, out=out)
    gi_attn.prefill(q, k, v, pos0, n_heads, n_kv, **kw)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        gi_attn.prefill(q, k, v, pos0, n_heads, n_kv, **kw)
    gen = torch.Generator(device=gpu)
    gen.manual_seed(6501)
    for r in range(3):
        say("widened prefill replay", r)
        q.copy_(torch.randn(q.shape, generator=gen, device=gpu))
        want = gi_attn.prefill(q, k, v, pos0, n_heads, n_kv, hd=hd, k_scale=ks, v_scale=vs, staged=False,
                               out_dtype=torch.float32)
        torch.cuda.synchronize()
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {r}"
