"""A prompt fed one token at a time through the split decode, as the reference's scripts/decode-accuracy.ps1 does
(GHOST_INFER_STEPWISE=1: every position of a ~1,500-token prompt goes through the split-context decode attention,
checked against the exact CPU path). Here token b's decode call attends to keys 0..b of the prompt's own cache, and
the 1,500 rows, stacked, are held to float64 causal attention over the whole prompt at the split path's bar. The slice
plan changes with the span (one slice, then more of them as it grows), so every plan the span passes through is
exercised, with one workspace reused throughout."""
import sys

import numpy as np
import pytest
import torch

import gi_attn
from attn_common import assert_close, make_inputs, make_inputs_i8, reference_f64, reference_f64_i8, split_f64_tol

pytestmark = pytest.mark.gpu

N = 1500


@pytest.mark.parametrize("fmt,n_heads,n_kv,hd", [("f16", 8, 2, 128), ("i8", 8, 2, 128), ("f16", 9, 3, 64),
                                                  ("i8", 16, 2, 256), ("f16", 8, 8, 80)])
def test_stepwise_prompt(gpu, fmt, n_heads, n_kv, hd):
    print("[case] stepwise", fmt, n_heads, n_kv, hd, flush=True)
    sys.stdout.flush()
    if fmt == "f16":
        q, k, v = make_inputs(4242, N, N, n_heads, n_kv, hd=hd)
        kt = torch.from_numpy(k.view(np.int16)).to(gpu).view(torch.float16)
        vt = torch.from_numpy(v.view(np.int16)).to(gpu).view(torch.float16)
        ks = vs = None
        want = reference_f64(q, k, v, 0, n_heads, n_kv, hd=hd)
    else:
        q, k, v, ksn, vsn = make_inputs_i8(4243, N, N, n_heads, n_kv, hd=hd)
        kt, vt, ks, vs = (torch.from_numpy(x).to(gpu) for x in (k, v, ksn, vsn))
        want = reference_f64_i8(q, k, v, ksn, vsn, 0, n_heads, n_kv, hd=hd)
    qt = torch.from_numpy(q).to(gpu)
    out = torch.empty((N, n_heads * hd), dtype=torch.float32, device=gpu)
    ws = gi_attn.new_workspace(N, 1, n_heads, n_kv, hd=hd, device=gpu)
    for b in range(N):
        gi_attn.decode(qt[b:b + 1], kt, vt, b, n_heads, n_kv, hd=hd, out=out[b:b + 1], workspace=ws, k_scale=ks,
                       v_scale=vs)
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), want, *split_f64_tol(fmt, hd), what=f"stepwise {fmt} hd {hd}")
