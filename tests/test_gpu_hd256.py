"""Parity of head size 256 (the reference's wide heads, src/cuda.rs:1762-1781 and attention_prefill_tc256
src/cuda.rs:2623) on the gfx950 kernels, through the C ABI.

Bar: max-abs 2e-3 and relative L2 1e-3 against the oracle's Model::attention (src/model.rs:1320-1409, any
head size), and 2e-5 against float64 attention for decode (f32 scores and probabilities, as at head
size 128).
"""
import sys

import numpy as np
import pytest
import torch

import gi_attn
import gi_oracle as O
from attn_common import assert_close, make_inputs, reference_f64

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
    # variant (1 and 2 column blocks, the shared-slice variant), G = 3
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
