"""Writes the small golden fixtures of the attention path: seeded inputs and float64 expected outputs.

    python tests/golden/make_golden.py

The expected outputs come from the textbook causal softmax attention in float64
(tests/attn_common.reference_f64), not from the oracle under test. Inputs follow the configs' recipe
(Q N(0,1), K/V N(0,1) rounded to f16, scale 1/sqrt(128)) at sizes small enough to commit.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
from attn_common import make_inputs, reference_f64  # noqa: E402

CASES = {
    # name: (seed, n_tok, pos0, n_heads, n_kv, q dtype)
    "decode_g4_ctx64": (101, 1, 63, 32, 8, np.float32),
    "decode_g8_ctx300": (102, 1, 299, 32, 4, np.float32),
    "verify_8tok_ctx136": (103, 8, 128, 32, 4, np.float32),
    "prefill_48tok": (104, 48, 0, 8, 2, np.float16),
    "prefill_chunk_32at64": (105, 32, 64, 8, 2, np.float16),
}


def main():
    for name, (seed, n_tok, pos0, n_heads, n_kv, qd) in CASES.items():
        q, k, v = make_inputs(seed, n_tok, pos0 + n_tok, n_heads, n_kv, q_dtype=qd)
        out = reference_f64(q, k, v, pos0, n_heads, n_kv).astype(np.float32)
        np.savez_compressed(os.path.join(HERE, name + ".npz"), q=q, k=k, v=v, out=out, pos0=pos0,
                            n_heads=n_heads, n_kv=n_kv)
        print(name, q.shape, k.shape)


if __name__ == "__main__":
    main()
