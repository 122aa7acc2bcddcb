"""Shared helpers of the attention tests: seeded inputs and an independent float64 reference."""
import numpy as np

# The north star's parity bar on f32 outputs.
MAX_ABS_TOL = 2e-3
REL_L2_TOL = 1e-3


def make_inputs(seed, n_tok, ctx, n_heads, n_kv, hd=128, q_dtype=np.float32):
    """Seeded N(0,1) inputs: q [n_tok, n_heads*hd] (q_dtype), K/V cache f16 bits [ctx, n_kv*hd] (uint16).
    One generator per tensor: seed, seed + 1, seed + 2."""
    q = np.random.default_rng(seed).standard_normal((n_tok, n_heads * hd), dtype=np.float32)
    if q_dtype == np.float16:
        q = q.astype(np.float16)
    k = np.random.default_rng(seed + 1).standard_normal((ctx, n_kv * hd), dtype=np.float32).astype(np.float16)
    v = np.random.default_rng(seed + 2).standard_normal((ctx, n_kv * hd), dtype=np.float32).astype(np.float16)
    return q, k.view(np.uint16), v.view(np.uint16)


def f16_values(bits):
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float64)


def reference_f64(q, kbits, vbits, pos0, n_heads, n_kv, hd=128, scale=None):
    """Textbook causal softmax attention in float64: token b attends to keys 0..pos0+b."""
    q = np.asarray(q, dtype=np.float64).reshape(q.shape[0], n_heads, hd)
    n = q.shape[0]
    k = f16_values(kbits).reshape(-1, n_kv, hd)
    v = f16_values(vbits).reshape(-1, n_kv, hd)
    if scale is None:
        scale = 1.0 / np.sqrt(hd)
    G = n_heads // n_kv
    out = np.zeros((n, n_heads, hd))
    for kvh in range(n_kv):
        K = k[: pos0 + n, kvh]
        V = v[: pos0 + n, kvh]
        qh = q[:, kvh * G:(kvh + 1) * G]  # [n, G, hd]
        s = np.einsum("ngd,td->ngt", qh, K) * scale
        mask = np.arange(pos0 + n)[None, :] > (pos0 + np.arange(n))[:, None]
        s = np.where(mask[:, None, :], -np.inf, s)
        s -= s.max(axis=-1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(axis=-1, keepdims=True)
        out[:, kvh * G:(kvh + 1) * G] = np.einsum("ngt,td->ngd", p, V)
    return out.reshape(n, n_heads * hd)


def errors(got, want):
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    diff = got - want
    max_abs = float(np.abs(diff).max()) if diff.size else 0.0
    rel = float(np.linalg.norm(diff) / max(np.linalg.norm(want), 1e-300))
    return max_abs, rel


def assert_close(got, want, max_abs=MAX_ABS_TOL, rel_l2=REL_L2_TOL, what=""):
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    ma, rl = errors(got, want)
    assert ma <= max_abs and rl <= rel_l2, f"{what}: max_abs {ma:.3g} (tol {max_abs}), rel_l2 {rl:.3g} (tol {rel_l2})"
    return ma, rl
