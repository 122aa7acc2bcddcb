"""Writes the small golden fixtures of the attention path: seeded inputs and float64 expected outputs.

    python tests/golden/make_golden.py [NAME ...]   (no names: every case)

The expected outputs come from the textbook causal softmax attention in float64
(tests/attn_common.reference_f64, over the dequantised cache for int8 and the 4-bit cache), not from the oracle
under test. Inputs follow the configs' recipe (Q N(0,1), K/V N(0,1) rounded to f16, scale 1/sqrt(head size)) at
sizes small enough to commit; the int8 cases hold int8 rows and their f32 scales (keys ks, vs); the 4-bit cases
(key q4 = 1) hold rows of 128 nibble-pair bytes and their f16 scale bits, 8 a row (ks, vs as uint16).
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
from attn_common import (make_inputs, make_inputs_i8, make_inputs_q4, reference_f64, reference_f64_i8,  # noqa: E402
                         reference_f64_q4)

CASES = {
    # name: (seed, n_tok, pos0, n_heads, n_kv, q dtype, head size, cache: False f16, True int8, "q4" 4-bit)
    "decode_g4_ctx64": (101, 1, 63, 32, 8, np.float32, 128, False),
    "decode_g8_ctx300": (102, 1, 299, 32, 4, np.float32, 128, False),
    "verify_8tok_ctx136": (103, 8, 128, 32, 4, np.float32, 128, False),
    "prefill_48tok": (104, 48, 0, 8, 2, np.float16, 128, False),
    "prefill_chunk_32at64": (105, 32, 64, 8, 2, np.float16, 128, False),
    "decode_h256_ctx200": (106, 1, 199, 16, 2, np.float32, 256, False),
    "prefill_h256_40tok": (107, 40, 0, 4, 1, np.float16, 256, False),
    "decode_i8_g8_ctx300": (108, 1, 299, 32, 4, np.float32, 128, True),
    "verify_i8_4tok_ctx100": (109, 4, 96, 16, 2, np.float32, 128, True),
    "decode_h256_i8_ctx200": (110, 1, 199, 16, 2, np.float32, 256, True),
    "verify_h256_i8_3tok_ctx90": (111, 3, 87, 16, 2, np.float32, 256, True),
    "prefill_h256_i8_40tok": (112, 40, 0, 4, 1, np.float32, 256, True),
    "decode_h256_q4_ctx200": (113, 1, 199, 16, 2, np.float32, 256, "q4"),
    "verify_h256_q4_3tok_ctx90": (114, 3, 87, 16, 2, np.float32, 256, "q4"),
    "prefill_h256_q4_40tok": (115, 40, 0, 4, 1, np.float32, 256, "q4"),
    # head size 64 at SmolLM2-135M's 9 query / 3 kv heads (the reference's attention_prefill_tc64 and its split
    # decode at head size 64)
    "decode_h64_smollm2_ctx300": (116, 1, 299, 9, 3, np.float32, 64, False),
    "verify_h64_smollm2_5tok_ctx130": (117, 5, 125, 9, 3, np.float32, 64, False),
    "prefill_h64_smollm2_48tok": (118, 48, 0, 9, 3, np.float16, 64, False),
    "decode_h64_i8_smollm2_ctx300": (119, 1, 299, 9, 3, np.float32, 64, True),
    "prefill_h64_i8_smollm2_40tok": (120, 40, 0, 9, 3, np.float32, 64, True),
    # the f32 kernels' head sizes: Phi-2-style 80 and Phi-3-style 96 (the reference's f32 fallback kernels)
    "decode_h80_ctx300": (121, 1, 299, 4, 4, np.float32, 80, False),
    "verify_h96_i8_4tok_ctx100": (122, 4, 96, 12, 4, np.float32, 96, True),
    "prefill_h96_48tok": (123, 48, 0, 8, 8, np.float16, 96, False),
    "prefill_h80_i8_40tok": (124, 40, 0, 8, 2, np.float32, 80, True),
}


def main():
    names = sys.argv[1:] or list(CASES)
    for name in names:
        seed, n_tok, pos0, n_heads, n_kv, qd, hd, i8 = CASES[name]
        extra = {}
        if i8 == "q4":  # random nibbles with f16 scales near 1/4, dequantised values of standard deviation ~1
            q, k, v, ks, vs = make_inputs_q4(seed, n_tok, pos0 + n_tok, n_heads, n_kv)
            out = reference_f64_q4(q, k, v, ks, vs, pos0, n_heads, n_kv).astype(np.float32)
            extra = {"ks": ks, "vs": vs, "q4": 1}
        elif i8:  # int8 rows round(40 N(0,1)) with f32 scales near 1/40, as quantised N(0,1) rows
            q, k, v, ks, vs = make_inputs_i8(seed, n_tok, pos0 + n_tok, n_heads, n_kv, hd=hd)
            out = reference_f64_i8(q, k, v, ks, vs, pos0, n_heads, n_kv, hd=hd).astype(np.float32)
            extra = {"ks": ks, "vs": vs}
        else:
            q, k, v = make_inputs(seed, n_tok, pos0 + n_tok, n_heads, n_kv, hd=hd, q_dtype=qd)
            out = reference_f64(q, k, v, pos0, n_heads, n_kv, hd=hd).astype(np.float32)
        np.savez_compressed(os.path.join(HERE, name + ".npz"), q=q, k=k, v=v, out=out, pos0=pos0,
                            n_heads=n_heads, n_kv=n_kv, hd=hd, **extra)
        print(name, q.shape, k.shape)


if __name__ == "__main__":
    main()
