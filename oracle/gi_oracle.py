"""ctypes wrapper of the CPU oracle (libgi_oracle.so). Test infrastructure only: imported by tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg, never by the product path.

Each function names the reference code it restates; gi_oracle.cpp's header lists how each is pinned.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libgi_oracle.so")

_lib = None


def build():
    subprocess.run(["make", "-s", "-B", "-C", HERE, "libgi_oracle.so"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        vp, i, l, f = ctypes.c_void_p, ctypes.c_int, ctypes.c_long, ctypes.c_float
        L.gio_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.gio_f16_to_f32.restype = f
        L.gio_f32_to_f16.argtypes = [f]
        L.gio_f32_to_f16.restype = ctypes.c_uint16
        L.gio_f16_to_f32_array.argtypes = [vp, vp, ctypes.c_size_t]
        L.gio_f32_to_f16_array.argtypes = [vp, vp, ctypes.c_size_t]
        L.gio_dot_f32.argtypes = [vp, vp, i]
        L.gio_dot_f32.restype = f
        L.gio_att_want.argtypes = [i]
        L.gio_att_want.restype = i
        L.gio_att_chunk.argtypes = [i, i, i]
        L.gio_att_chunk.restype = i
        L.gio_max_splits.argtypes = [i, i, i]
        L.gio_max_splits.restype = i
        L.gio_attention_f32.argtypes = [vp, l, vp, vp, l, vp, l, i, i, i, i, i, f, i]
        L.gio_attention_f16kv.argtypes = [vp, l, vp, vp, l, vp, l, i, i, i, i, i, f, i]
        L.gio_decode_gpu.argtypes = [vp, l, vp, vp, l, vp, l, i, i, i, i, f, i, i, i, i]
        L.gio_prefill_tc.argtypes = [vp, l, vp, vp, l, vp, l, i, i, i, i, f, i]
        L.gio_qk_norm_rope.argtypes = [vp, vp, vp, vp, vp, l, l, i, i, i, i, i, i, f, vp, i, f]
        L.gio_qk_norm_rope_i8.argtypes = [vp, vp, vp, vp, vp, vp, vp, l, l, l, l, i, i, i, i, i, i, f, vp, i, f]
        L.gio_decode_gpu_i8.argtypes = [vp, l, vp, vp, vp, vp, l, vp, l, i, i, i, i, f, i, i, i, i]
        L.gio_decode_tc256_i8.argtypes = [vp, l, vp, vp, vp, vp, l, vp, l, i, i, i, i, f, i, i, i, i]
        L.gio_kv_quant_i8.argtypes = [vp, l, i, vp, vp]
        L.gio_prefill_tc_i8.argtypes = [vp, l, vp, vp, vp, vp, l, vp, l, i, i, i, i, f, i]
        L.gio_prefill_tc256.argtypes = [vp, l, vp, vp, l, vp, l, i, i, i, i, f, i]
        L.gio_prefill_tc64.argtypes = [vp, l, vp, vp, l, vp, l, i, i, i, i, f, i]
        L.gio_prefill_tc64_i8.argtypes = [vp, l, vp, vp, vp, vp, l, vp, l, i, i, i, i, f, i]
        L.gio_prefill_tc256_i8.argtypes = [vp, l, vp, vp, vp, vp, l, vp, l, i, i, i, i, f, i]
        L.gio_kv4_fwht.argtypes = [vp, l]
        L.gio_kv4_quant.argtypes = [vp, l, vp, vp]
        L.gio_kv4_dequant.argtypes = [vp, vp, l, i, vp]
        L.gio_qk_norm_rope_q4.argtypes = [vp, vp, vp, vp, vp, vp, vp, i, i, i, i, i, f, vp, i, f]
        L.gio_decode_tc256_q4.argtypes = [vp, l, vp, vp, vp, vp, l, vp, l, i, i, i, i, f, i, i, i, i]
        L.gio_prefill_tc256_q4.argtypes = [vp, l, vp, vp, vp, vp, l, vp, l, i, i, i, i, f, i]
        _lib = L
    return _lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def f16_bits_to_f32(bits):
    """src/quant.rs:10-32 over an array of uint16 bit patterns."""
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(bits.shape, dtype=np.float32)
    lib().gio_f16_to_f32_array(_p(bits), _p(out), bits.size)
    return out


def f32_to_f16_bits(x):
    """src/quant.rs:34-60 (round to nearest even) over an array."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().gio_f32_to_f16_array(_p(x), _p(out), x.size)
    return out


def dot_f32(a, b):
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    return lib().gio_dot_f32(_p(a), _p(b), a.size)


def att_want(n_kv):
    return lib().gio_att_want(n_kv)


def att_chunk(span, want, cap=128):
    return lib().gio_att_chunk(span, want, cap)


def max_splits(ctx, want, cap=128):
    return lib().gio_max_splits(ctx, want, cap)


def _rows(a, dtype):
    a = np.ascontiguousarray(a, dtype=dtype)
    return a.reshape(a.shape[0], -1)


def attention(q, kc, vc, pos0, n_heads, n_kv, hd=128, scale=None, threads=8):
    """Model::attention (src/model.rs:1320-1409). q: f32 [n, n_heads*hd]; kc/vc: [pos, n_kv*hd] as f32
    values or as f16 bit patterns (uint16, widened exactly). Returns f32 [n, n_heads*hd]."""
    q = _rows(q, np.float32)
    n = q.shape[0]
    if scale is None:
        scale = 1.0 / np.sqrt(hd)
    out = np.zeros((n, n_heads * hd), dtype=np.float32)
    if kc.dtype == np.uint16:
        kc, vc = _rows(kc, np.uint16), _rows(vc, np.uint16)
        fn = lib().gio_attention_f16kv
    else:
        kc, vc = _rows(kc, np.float32), _rows(vc, np.float32)
        fn = lib().gio_attention_f32
    assert kc.shape[0] >= pos0 + n and kc.shape[1] == n_kv * hd
    fn(_p(q), q.shape[1], _p(kc), _p(vc), kc.shape[1], _p(out), out.shape[1], pos0, n, n_heads, n_kv, hd, scale,
       threads)
    return out


def decode_gpu_semantics(q, kc, vc, pos0, n_heads, n_kv, scale=None, cap=128, threads=8):
    """attention_partial_gqa + attention_combine (src/cuda.rs:1684-1865, 2806-2836) with the host's
    split arithmetic (src/cuda.rs:8426-8444, 8506-8511). kc/vc: uint16 f16 bits [pos, n_kv*128]."""
    q = _rows(q, np.float32)
    m = q.shape[0]
    kc, vc = _rows(kc, np.uint16), _rows(vc, np.uint16)
    if scale is None:
        scale = 1.0 / np.sqrt(128)
    want = att_want(n_kv)
    nsplit = max(-(-span // att_chunk(span, want, cap)) for span in range(pos0 + 1, pos0 + m + 1))
    out = np.zeros((m, n_heads * 128), dtype=np.float32)
    lib().gio_decode_gpu(_p(q), q.shape[1], _p(kc), _p(vc), kc.shape[1], _p(out), out.shape[1], pos0, m, n_heads,
                         n_kv, scale, nsplit, want, cap, threads)
    return out


def decode_gpu_semantics_i8(q, kc, vc, ks, vs, pos0, n_heads, n_kv, scale=None, cap=128, threads=8):
    """attention_partial_gqa + attention_combine over the KV8 cache (src/cuda.rs:209-226, 1684-1865, 2806-2836).
    kc/vc: int8 [pos, n_kv*128]; ks/vs: f32 scales [pos, n_kv]."""
    q = _rows(q, np.float32)
    m = q.shape[0]
    kc, vc = _rows(kc, np.int8), _rows(vc, np.int8)
    ks, vs = _rows(ks, np.float32), _rows(vs, np.float32)
    assert ks.shape == (kc.shape[0], n_kv) and vs.shape == ks.shape
    if scale is None:
        scale = 1.0 / np.sqrt(128)
    want = att_want(n_kv)
    nsplit = max(-(-span // att_chunk(span, want, cap)) for span in range(pos0 + 1, pos0 + m + 1))
    out = np.zeros((m, n_heads * 128), dtype=np.float32)
    lib().gio_decode_gpu_i8(_p(q), q.shape[1], _p(kc), _p(vc), _p(ks), _p(vs), kc.shape[1], _p(out), out.shape[1],
                            pos0, m, n_heads, n_kv, scale, nsplit, want, cap, threads)
    return out


def decode_tc256_i8(q, kc, vc, ks, vs, pos0, n_heads, n_kv, scale=None, cap=128, threads=8, want=None):
    """attention_decode_tc256 over the KV8 cache (src/cuda.rs:2625-2802) + attention_combine (src/cuda.rs:2806-2836),
    with the host's split arithmetic (src/cuda.rs:8426-8444). kc/vc int8 [pos, n_kv*256]; ks/vs f32 [pos, n_kv]."""
    q = _rows(q, np.float32)
    m = q.shape[0]
    kc, vc = _rows(kc, np.int8), _rows(vc, np.int8)
    ks, vs = _rows(ks, np.float32), _rows(vs, np.float32)
    assert ks.shape == (kc.shape[0], n_kv) and vs.shape == ks.shape and kc.shape[1] == n_kv * 256
    if scale is None:
        scale = 1.0 / 16.0
    want = att_want(n_kv) if want is None else want
    nsplit = max(-(-span // att_chunk(span, want, cap)) for span in range(pos0 + 1, pos0 + m + 1))
    out = np.zeros((m, n_heads * 256), dtype=np.float32)
    lib().gio_decode_tc256_i8(_p(q), q.shape[1], _p(kc), _p(vc), _p(ks), _p(vs), kc.shape[1], _p(out), out.shape[1],
                              pos0, m, n_heads, n_kv, scale, nsplit, want, cap, threads)
    return out


def kv_quant_i8(x):
    """kv_store with KV8 (src/cuda.rs:333-339) over rows of x (f32 [..., hd]): returns (int8 rows, f32 scales)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    hd = x.shape[-1]
    rows = x.size // hd
    q = np.empty(x.shape, dtype=np.int8)
    sc = np.empty(x.shape[:-1], dtype=np.float32)
    lib().gio_kv_quant_i8(_p(x), rows, hd, _p(q), _p(sc))
    return q, sc


def kv4_fwht(x):
    """kv4_fwht (src/cuda.rs:242-256) over rows of 256 values: the normalized Walsh-Hadamard transform, Sylvester
    order, in the reference's butterfly order (also hadamard_rows with block 256, src/cuda.rs:4675-4693)."""
    x = np.array(x, dtype=np.float32, order="C", copy=True)
    assert x.shape[-1] == 256
    lib().gio_kv4_fwht(_p(x), x.size // 256)
    return x


def kv4_quant(x):
    """kv_store with KV4 (src/cuda.rs:340-357) over already-rotated rows of 256 values: returns (uint8 [..., 128]
    nibble pairs, uint16 [..., 8] f16 scale bits)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    assert x.shape[-1] == 256
    rows = x.size // 256
    q = np.empty(x.shape[:-1] + (128,), dtype=np.uint8)
    sc = np.empty(x.shape[:-1] + (8,), dtype=np.uint16)
    lib().gio_kv4_quant(_p(x), rows, _p(q), _p(sc))
    return q, sc


def kv4_dequant(c, sc, n_kv):
    """The f16 values (uint16 bits, [rows, n_kv*256]) the tensor-core kernels use for a 4-bit cache
    (kv4_pair, src/cuda.rs:238-240): f16((n - 8) * scale). c: uint8 [rows, n_kv*128]; sc: uint16 [rows, n_kv*8]."""
    c = np.ascontiguousarray(c, dtype=np.uint8).reshape(-1, n_kv * 128)
    sc = np.ascontiguousarray(sc, dtype=np.uint16).reshape(-1, n_kv * 8)
    out = np.empty((c.shape[0], n_kv * 256), dtype=np.uint16)
    lib().gio_kv4_dequant(_p(c), _p(sc), c.shape[0], n_kv, _p(out))
    return out


def qk_norm_rope_q4(qkv, kc, vc, ks, vs, pos0, n_heads, n_kv, rope_dim=None, base=10000.0, qn=None, kn=None, ff=None,
                    neox=True, eps=1e-6):
    """qk_norm_rope with the KV4 build (src/cuda.rs:437-486, 340-357): q and k heads rotated after RoPE (written
    back rotated), k rows quantised, v rows rotated then quantised. Head size 256; caches in the reference layout:
    kc/vc uint8 [pos, n_kv*128], ks/vs uint16 f16 bits [pos, n_kv*8]. Returns (qkv, kc, vc, ks, vs) copies."""
    qkv = np.array(qkv, dtype=np.float32, order="C", copy=True)
    kc = np.array(kc, dtype=np.uint8, order="C", copy=True)
    vc = np.array(vc, dtype=np.uint8, order="C", copy=True)
    ks = np.array(ks, dtype=np.uint16, order="C", copy=True)
    vs = np.array(vs, dtype=np.uint16, order="C", copy=True)
    n = qkv.shape[0]
    rope_dim = 256 if rope_dim is None else rope_dim
    opts = [None if a is None else np.ascontiguousarray(a, dtype=np.float32) for a in (qn, kn, ff)]
    ptrs = [None if a is None else _p(a) for a in opts]
    lib().gio_qk_norm_rope_q4(_p(qkv), ptrs[0], ptrs[1], _p(kc), _p(vc), _p(ks), _p(vs), pos0, n, n_heads, n_kv,
                              rope_dim, base, ptrs[2], 1 if neox else 0, eps)
    return qkv, kc, vc, ks, vs


def decode_tc256_q4(q, kc, vc, ks, vs, pos0, n_heads, n_kv, scale=None, cap=128, threads=8, want=None):
    """attention_decode_tc256 with the KV4 build (src/cuda.rs:2681-2760) + attention_combine, over rotated queries:
    the output is rotated (kv4_fwht turns it back, as hadamard_rows does). kc/vc uint8 [pos, n_kv*128], ks/vs
    uint16 [pos, n_kv*8]."""
    q = _rows(q, np.float32)
    m = q.shape[0]
    kc, vc = _rows(kc, np.uint8), _rows(vc, np.uint8)
    ks, vs = _rows(ks, np.uint16), _rows(vs, np.uint16)
    assert kc.shape[1] == n_kv * 128 and ks.shape == (kc.shape[0], n_kv * 8) and vs.shape == ks.shape
    assert kc.shape[0] >= pos0 + m
    if scale is None:
        scale = 1.0 / 16.0
    want = att_want(n_kv) if want is None else want
    nsplit = max(-(-span // att_chunk(span, want, cap)) for span in range(pos0 + 1, pos0 + m + 1))
    out = np.zeros((m, n_heads * 256), dtype=np.float32)
    lib().gio_decode_tc256_q4(_p(q), q.shape[1], _p(kc), _p(vc), _p(ks), _p(vs), kc.shape[0], _p(out), out.shape[1],
                              pos0, m, n_heads, n_kv, scale, nsplit, want, cap, threads)
    return out


def prefill_tc256_q4(q, kc, vc, ks, vs, pos0, n_heads, n_kv, scale=None, threads=8):
    """attention_prefill_tc256 with the KV4 build (src/cuda.rs:2495-2514): the f16 cache's arithmetic over the
    4-bit cache's f16 values. Rotated queries in, rotated output out."""
    q = _rows(q, np.float32)
    n = q.shape[0]
    kc, vc = _rows(kc, np.uint8), _rows(vc, np.uint8)
    ks, vs = _rows(ks, np.uint16), _rows(vs, np.uint16)
    assert kc.shape[1] == n_kv * 128 and ks.shape == (kc.shape[0], n_kv * 8) and kc.shape[0] >= pos0 + n
    if scale is None:
        scale = 1.0 / 16.0
    out = np.zeros((n, n_heads * 256), dtype=np.float32)
    lib().gio_prefill_tc256_q4(_p(q), q.shape[1], _p(kc), _p(vc), _p(ks), _p(vs), kc.shape[0], _p(out), out.shape[1],
                               pos0, n, n_heads, n_kv, scale, threads)
    return out


def prefill_tc_semantics(q, kc, vc, pos0, n_heads, n_kv, scale=None, threads=8, hd=128):
    """attn_prefill_tc<128> (src/cuda.rs:2408-2617): f16-rounded Q*scale*log2(e) and P; hd=256 follows
    attention_prefill_tc256 (src/cuda.rs:2623) and hd=64 attention_prefill_tc64 (src/cuda.rs:2620), the same
    arithmetic."""
    q = _rows(q, np.float32)
    n = q.shape[0]
    kc, vc = _rows(kc, np.uint16), _rows(vc, np.uint16)
    if scale is None:
        scale = 1.0 / np.sqrt(hd)
    out = np.zeros((n, n_heads * hd), dtype=np.float32)
    fn = {64: lib().gio_prefill_tc64, 128: lib().gio_prefill_tc, 256: lib().gio_prefill_tc256}[hd]
    fn(_p(q), q.shape[1], _p(kc), _p(vc), kc.shape[1], _p(out), out.shape[1], pos0, n, n_heads, n_kv, scale, threads)
    return out


def prefill_tc_semantics_i8(q, kc, vc, ks, vs, pos0, n_heads, n_kv, scale=None, threads=8, hd=128):
    """attn_prefill_tc<128> over the KV8 cache (src/cuda.rs:2408-2617 with KV8); hd=256 follows
    attention_prefill_tc256 (src/cuda.rs:2623) and hd=64 attention_prefill_tc64 (src/cuda.rs:2620). kc/vc int8
    [pos, n_kv*hd], ks/vs f32 [pos, n_kv]."""
    q = _rows(q, np.float32)
    n = q.shape[0]
    kc, vc = _rows(kc, np.int8), _rows(vc, np.int8)
    ks, vs = _rows(ks, np.float32), _rows(vs, np.float32)
    if scale is None:
        scale = 1.0 / np.sqrt(hd)
    out = np.zeros((n, n_heads * hd), dtype=np.float32)
    fn = {64: lib().gio_prefill_tc64_i8, 128: lib().gio_prefill_tc_i8, 256: lib().gio_prefill_tc256_i8}[hd]
    fn(_p(q), q.shape[1], _p(kc), _p(vc), _p(ks), _p(vs), kc.shape[1], _p(out), out.shape[1], pos0, n, n_heads, n_kv,
       scale, threads)
    return out


def qk_norm_rope(qkv, kc, vc, pos0, n_heads, n_kv, hd=128, rope_dim=None, base=10000.0, qn=None, kn=None, ff=None,
                 neox=True, eps=1e-6, kv_head_stride=None):
    """qk_norm_rope (src/cuda.rs:437-486) with an f16 cache: returns (qkv after norm and RoPE, kc, vc), the
    caches (uint16 f16 bits, rows of position t kv_stride elements apart) updated at positions pos0 ..
    pos0 + n - 1. Inputs are not modified."""
    qkv = np.array(qkv, dtype=np.float32, order="C", copy=True)
    kc = np.array(kc, dtype=np.uint16, order="C", copy=True)
    vc = np.array(vc, dtype=np.uint16, order="C", copy=True)
    n = qkv.shape[0]
    rope_dim = hd if rope_dim is None else rope_dim
    kv_stride = kc.strides[0] // 2
    kv_head_stride = hd if kv_head_stride is None else kv_head_stride
    opts = [None if a is None else np.ascontiguousarray(a, dtype=np.float32) for a in (qn, kn, ff)]
    ptrs = [None if a is None else _p(a) for a in opts]
    lib().gio_qk_norm_rope(_p(qkv), ptrs[0], ptrs[1], _p(kc), _p(vc), kv_stride, kv_head_stride, pos0, n, n_heads,
                           n_kv, hd, rope_dim, base, ptrs[2], 1 if neox else 0, eps)
    return qkv, kc, vc


def qk_norm_rope_i8(qkv, kc, vc, ks, vs, pos0, n_heads, n_kv, hd=128, rope_dim=None, base=10000.0, qn=None, kn=None,
                    ff=None, neox=True, eps=1e-6, kv_head_stride=None, sc_stride=None, sc_head_stride=1):
    """qk_norm_rope (src/cuda.rs:437-486) storing into an int8 cache (kv_store with KV8, src/cuda.rs:333-339).
    kc/vc: int8, rows of position t kv_stride elements apart; ks/vs: f32 scales, position t kv head h at
    t*sc_stride + h*sc_head_stride (default [pos][n_kv]). Returns (qkv, kc, vc, ks, vs) copies."""
    qkv = np.array(qkv, dtype=np.float32, order="C", copy=True)
    kc = np.array(kc, dtype=np.int8, order="C", copy=True)
    vc = np.array(vc, dtype=np.int8, order="C", copy=True)
    ks = np.array(ks, dtype=np.float32, order="C", copy=True)
    vs = np.array(vs, dtype=np.float32, order="C", copy=True)
    n = qkv.shape[0]
    rope_dim = hd if rope_dim is None else rope_dim
    kv_stride = kc.strides[0]
    kv_head_stride = hd if kv_head_stride is None else kv_head_stride
    sc_stride = n_kv if sc_stride is None else sc_stride
    opts = [None if a is None else np.ascontiguousarray(a, dtype=np.float32) for a in (qn, kn, ff)]
    ptrs = [None if a is None else _p(a) for a in opts]
    lib().gio_qk_norm_rope_i8(_p(qkv), ptrs[0], ptrs[1], _p(kc), _p(vc), _p(ks), _p(vs), kv_stride, kv_head_stride,
                              sc_stride, sc_head_stride, pos0, n, n_heads, n_kv, hd, rope_dim, base, ptrs[2],
                              1 if neox else 0, eps)
    return qkv, kc, vc, ks, vs
