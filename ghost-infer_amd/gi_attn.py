"""Python mirror of ghost-infer's attention operator over the gfx950 C ABI (include/gi_attn.h).

The reference's operator is GpuModel::attention (src/cuda.rs:8448-8541): for a layer it takes the
[q | k | v] f32 rows of the batch, the layer's f16 K/V cache, the session position and a verify
("exact") flag, and writes the f32 attention output. `attention()` keeps that contract; `decode()` and
`prefill()` expose the two kernels it dispatches to, with the shapes the benchmark configs name.

Tensors are torch CUDA tensors (torch is the device-memory and stream plumbing here; every computation
runs in the HIP kernels of libgi_attn.so). Work goes on torch's current stream. Errors raise
GiAttnError with the library's message, as the reference returns Err(String) from Api::check
(src/cuda.rs:5058-5068). There is no CPU fallback: without the built library every call raises.
"""
import ctypes
import math
import os

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libgi_attn.so")
HSACO_PATH = os.path.join(HERE, "gi_attn_gfx950.hsaco")

GI_F32 = 0
GI_F16 = 1
SPLIT_MAX_BATCH = 15  # src/cuda.rs:119
TILED_MIN_BATCH = 16  # src/cuda.rs:95

# Exported symbols of include/gi_attn.h
SYMBOLS = (
    "gi_init",
    "gi_last_error",
    "gi_attn_decode_plan",
    "gi_attn_decode_workspace_bytes",
    "gi_attn_decode",
    "gi_attn_decode_noalloc",
    "gi_attn_decode_i8",
    "gi_attn_decode_q4",
    "gi_attn_prefill",
    "gi_attn_prefill_i8",
    "gi_attention",
    "gi_attention_i8",
    "gi_attn_prefill_q4",
    "gi_attn_prefill_workspace_bytes",
    "gi_attn_prefill_f32",
    "gi_attn_prefill_i8_ws",
    "gi_attn_prefill_q4_ws",
    "gi_attention_q4",
    "gi_hadamard_rows",
    "gi_qk_norm_rope",
    "gi_qk_norm_rope_i8",
    "gi_qk_norm_rope_q4",
    "gi_kv_relayout",
    "gi_kernel_timing",
    "gi_kernel_timing_read",
)


class GiAttnError(RuntimeError):
    pass


_lib = None


def load_library(path=LIB_PATH):
    """Loads libgi_attn.so and declares its signatures (no GPU work)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise GiAttnError(f"{path} is not built: run ghost-infer_amd/gi_build.py (no fallback path exists)")
    lib = ctypes.CDLL(path)
    vp, i, ll, sz, f = ctypes.c_void_p, ctypes.c_int, ctypes.c_longlong, ctypes.c_size_t, ctypes.c_float
    lib.gi_init.argtypes = [ctypes.c_char_p]
    lib.gi_init.restype = i
    lib.gi_last_error.argtypes = []
    lib.gi_last_error.restype = ctypes.c_char_p
    lib.gi_attn_decode_plan.argtypes = [i, i, i, i, i, ctypes.POINTER(i), ctypes.POINTER(i)]
    lib.gi_attn_decode_plan.restype = i
    lib.gi_attn_decode_workspace_bytes.argtypes = [i, i, i, i, i]
    lib.gi_attn_decode_workspace_bytes.restype = sz
    lib.gi_kv_relayout.argtypes = [vp, vp, ll, ll, vp, ll, ll, i, i, i]
    lib.gi_kv_relayout.restype = i
    lib.gi_attn_decode.argtypes = [vp, vp, ll, vp, vp, ll, ll, vp, ll, vp, sz, i, vp, i, i, i, i, i, f]
    lib.gi_attn_decode.restype = i
    lib.gi_attn_decode_noalloc.argtypes = [vp, vp, ll, vp, vp, ll, ll, vp, ll, i, vp, i, i, i, i, i, f]
    lib.gi_attn_decode_noalloc.restype = i
    lib.gi_attn_decode_i8.argtypes = [vp, vp, ll, vp, vp, vp, vp, ll, ll, ll, ll, vp, ll, vp, sz, i, vp, i, i, i, i, i,
                                      f]
    lib.gi_attn_decode_i8.restype = i
    lib.gi_attn_decode_q4.argtypes = [vp, vp, ll, vp, vp, vp, vp, ll, ll, ll, ll, vp, ll, vp, sz, i, vp, i, i, i, i, f]
    lib.gi_attn_decode_q4.restype = i
    lib.gi_attn_prefill.argtypes = [vp, vp, i, ll, vp, vp, ll, ll, vp, i, ll, i, i, i, i, i, f]
    lib.gi_attn_prefill.restype = i
    lib.gi_attention.argtypes = [vp, vp, vp, vp, vp, vp, sz, i, vp, i, i, i, i, i, i]
    lib.gi_attention.restype = i
    lib.gi_attn_prefill_i8.argtypes = [vp, vp, i, ll, vp, vp, vp, vp, ll, ll, ll, ll, vp, i, ll, i, i, i, i, i, f]
    lib.gi_attn_prefill_i8.restype = i
    lib.gi_attention_i8.argtypes = [vp, vp, vp, vp, vp, vp, vp, vp, sz, i, vp, i, i, i, i, i, i]
    lib.gi_attention_i8.restype = i
    lib.gi_attn_prefill_q4.argtypes = [vp, vp, i, ll, vp, vp, vp, vp, ll, ll, ll, ll, vp, i, ll, i, i, i, i, f]
    lib.gi_attn_prefill_q4.restype = i
    lib.gi_attention_q4.argtypes = [vp, vp, vp, vp, vp, vp, vp, vp, sz, i, vp, i, i, i, i, i]
    lib.gi_attention_q4.restype = i
    lib.gi_attn_prefill_f32.argtypes = [vp, vp, i, ll, vp, vp, vp, vp, i, ll, ll, ll, ll, vp, i, ll, i, i, i, i, i, f]
    lib.gi_attn_prefill_f32.restype = i
    lib.gi_attn_prefill_workspace_bytes.argtypes = [i, i, i, i]
    lib.gi_attn_prefill_workspace_bytes.restype = sz
    lib.gi_attn_prefill_i8_ws.argtypes = [vp, vp, i, ll, vp, vp, vp, vp, ll, ll, ll, ll, vp, i, ll, i, i, i, i, i, f,
                                          vp, sz]
    lib.gi_attn_prefill_i8_ws.restype = i
    lib.gi_attn_prefill_q4_ws.argtypes = [vp, vp, i, ll, vp, vp, vp, vp, ll, ll, ll, ll, vp, i, ll, i, i, i, i, f, vp,
                                          sz]
    lib.gi_attn_prefill_q4_ws.restype = i
    lib.gi_hadamard_rows.argtypes = [vp, vp, ll, i, i]
    lib.gi_hadamard_rows.restype = i
    lib.gi_qk_norm_rope.argtypes = [vp, vp, vp, vp, vp, vp, ll, ll, i, vp, i, i, i, i, i, i, f, vp, i, f]
    lib.gi_qk_norm_rope.restype = i
    lib.gi_qk_norm_rope_i8.argtypes = [vp, vp, vp, vp, vp, vp, vp, vp, ll, ll, ll, ll, i, vp, i, i, i, i, i, i, f, vp,
                                       i, f]
    lib.gi_qk_norm_rope_i8.restype = i
    lib.gi_qk_norm_rope_q4.argtypes = [vp, vp, vp, vp, vp, vp, vp, vp, ll, ll, ll, ll, i, vp, i, i, i, i, i, f, vp, i,
                                       f]
    lib.gi_qk_norm_rope_q4.restype = i
    lib.gi_kernel_timing.argtypes = [i]
    lib.gi_kernel_timing.restype = i
    lib.gi_kernel_timing_read.argtypes = [ctypes.c_char_p, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(i)]
    lib.gi_kernel_timing_read.restype = i
    _lib = lib
    return lib


def _check(rc):
    if rc != 0:
        raise GiAttnError(load_library().gi_last_error().decode())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _need(t, name, dtype):
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise GiAttnError(f"{name} must be a CUDA tensor")
    if t.dtype != dtype:
        raise GiAttnError(f"{name} must be {dtype}, got {t.dtype}")
    if t.stride(-1) != 1:
        raise GiAttnError(f"{name} rows must be contiguous")


def _cache_layout(kc, vc, n_kv, hd, layout, dtypes=(torch.float16,)):
    """(kv_stride, kv_head_stride, capacity) of a cache pair.

    layout "reference": [capacity, n_kv, hd] (or [capacity, n_kv*hd]), as the reference keeps it
    (src/cuda.rs:365-369); "head_major": [n_kv, capacity, hd], each kv head's rows contiguous. The caches
    are f16, or int8 where dtypes allows it (with f32 scales, see _scale_layout)."""
    if kc.dtype not in dtypes:
        raise GiAttnError(f"k_cache must be one of {dtypes}, got {kc.dtype}")
    for t, name in ((kc, "k_cache"), (vc, "v_cache")):
        _need(t, name, kc.dtype)
        if not t.is_contiguous():
            raise GiAttnError(f"{name} must be contiguous")
    if kc.shape != vc.shape:
        raise GiAttnError("k_cache and v_cache shapes differ")
    if layout == "reference":
        if kc.numel() % (n_kv * hd):
            raise GiAttnError(f"cache of shape {tuple(kc.shape)} is not [capacity, {n_kv}, {hd}]")
        return n_kv * hd, hd, kc.numel() // (n_kv * hd)
    if layout == "head_major":
        if kc.dim() != 3 or kc.shape[0] != n_kv or kc.shape[2] != hd:
            raise GiAttnError(f"head-major cache must be [{n_kv}, capacity, {hd}], got {tuple(kc.shape)}")
        return hd, kc.shape[1] * hd, kc.shape[1]
    raise GiAttnError(f"unknown cache layout {layout!r}")


def _scale_layout(ks, vs, n_kv, capacity, layout):
    """(sc_stride, sc_head_stride) of an int8 cache's f32 scales: [capacity, n_kv] with the reference layout
    (kv_store's KV_SROWP, src/cuda.rs:365-369), [n_kv, capacity] with the head-major one."""
    for t, name in ((ks, "k_scale"), (vs, "v_scale")):
        if t is None:
            raise GiAttnError(f"an int8 cache needs {name}")
        _need(t, name, torch.float32)
        if not t.is_contiguous():
            raise GiAttnError(f"{name} must be contiguous")
    want = (capacity, n_kv) if layout == "reference" else (n_kv, capacity)
    if tuple(ks.shape) != want or tuple(vs.shape) != want:
        raise GiAttnError(f"scales must be {list(want)}, got {tuple(ks.shape)} and {tuple(vs.shape)}")
    return (n_kv, 1) if layout == "reference" else (1, capacity)


def _q4_layout(kc, vc, ks, vs, n_kv, layout):
    """(kv_stride, kv_head_stride, sc_stride, sc_head_stride, capacity) of a 4-bit cache (head size 256): uint8
    rows of 128 bytes and float16 scales, 8 a row. layout "reference": [capacity, n_kv, 128] and [capacity, n_kv,
    8] (src/cuda.rs:365-369's KV_ROWP / KV_SROWP with KV4); "head_major": [n_kv, capacity, 128] and [n_kv,
    capacity, 8]. Strides of the rows in bytes, of the scales in f16 elements."""
    for t, name, dt in ((kc, "k_cache", torch.uint8), (vc, "v_cache", torch.uint8), (ks, "k_scale", torch.float16),
                        (vs, "v_scale", torch.float16)):
        if t is None:
            raise GiAttnError(f"a 4-bit cache needs {name}")
        _need(t, name, dt)
        if not t.is_contiguous():
            raise GiAttnError(f"{name} must be contiguous")
    if kc.shape != vc.shape or ks.shape != vs.shape:
        raise GiAttnError("k and v shapes differ")
    if layout == "reference":
        if kc.numel() % (n_kv * 128):
            raise GiAttnError(f"cache of shape {tuple(kc.shape)} is not [capacity, {n_kv}, 128]")
        cap = kc.numel() // (n_kv * 128)
        if ks.numel() != cap * n_kv * 8:
            raise GiAttnError(f"scales must be [{cap}, {n_kv}, 8], got {tuple(ks.shape)}")
        return n_kv * 128, 128, n_kv * 8, 8, cap
    if layout == "head_major":
        if kc.dim() != 3 or kc.shape[0] != n_kv or kc.shape[2] != 128:
            raise GiAttnError(f"head-major cache must be [{n_kv}, capacity, 128], got {tuple(kc.shape)}")
        cap = kc.shape[1]
        if tuple(ks.shape) != (n_kv, cap, 8):
            raise GiAttnError(f"head-major scales must be [{n_kv}, {cap}, 8], got {tuple(ks.shape)}")
        return 128, cap * 128, 8, cap * 8, cap
    raise GiAttnError(f"unknown cache layout {layout!r}")


def init(code_object_path=None):
    """Loads the code object on the current device (optional: the first call does it)."""
    lib = load_library()
    _check(lib.gi_init(code_object_path.encode() if code_object_path else None))


def decode_plan(max_span, n_tok, n_heads, n_kv, hd=128):
    """(keys per slice, slices per token) of a decode call; counterpart of att_chunk/max_splits."""
    lib = load_library()
    chunk, nsplit = ctypes.c_int(), ctypes.c_int()
    _check(lib.gi_attn_decode_plan(max_span, n_tok, n_heads, n_kv, hd, ctypes.byref(chunk), ctypes.byref(nsplit)))
    return chunk.value, nsplit.value


def workspace_bytes(ctx_cap, n_tok, n_heads, n_kv, hd=128):
    """Workspace bytes of decode calls of up to n_tok tokens with spans up to ctx_cap."""
    return int(load_library().gi_attn_decode_workspace_bytes(ctx_cap, n_tok, n_heads, n_kv, hd))


def new_workspace(ctx_cap, n_tok, n_heads, n_kv, hd=128, device="cuda"):
    """A decode workspace (uninitialised: every call writes the partials it reads)."""
    nbytes = workspace_bytes(ctx_cap, n_tok, n_heads, n_kv, hd)
    return torch.empty((nbytes + 3) // 4, dtype=torch.float32, device=device)


def decode(q, k_cache, v_cache, pos0, n_heads, n_kv, hd=128, scale=None, out=None, workspace=None, posp=None,
           ctx_cap=0, kv_layout="reference", k_scale=None, v_scale=None):
    """Decode/verify attention of n_tok = q.shape[0] tokens at positions pos0.. (causal within the block).

    q: f32 [n_tok, >= n_heads*hd] (row stride q.stride(0)); caches f16, or int8 with f32 k_scale / v_scale
    (the reference's KV8 cache), in kv_layout (see _cache_layout, _scale_layout); returns f32
    [n_tok, n_heads*hd]. posp: an int32 CUDA tensor holding the position (graph replay), with ctx_cap the
    largest span the launch shape must cover.
    """
    _need(q, "q", torch.float32)
    kv_stride, kv_head_stride, capacity = _cache_layout(k_cache, v_cache, n_kv, hd, kv_layout,
                                                        (torch.float16, torch.int8))
    i8 = k_cache.dtype == torch.int8
    if i8:
        sc_stride, sc_head_stride = _scale_layout(k_scale, v_scale, n_kv, capacity, kv_layout)
    n_tok = q.shape[0]
    if scale is None:
        scale = 1.0 / math.sqrt(hd)
    if out is None:
        out = torch.empty((n_tok, n_heads * hd), dtype=torch.float32, device=q.device)
    _need(out, "out", torch.float32)
    if posp is not None:
        _need(posp, "posp", torch.int32)
    need_rows = ctx_cap if posp is not None else pos0 + n_tok
    if capacity < need_rows:
        raise GiAttnError(f"the cache holds {capacity} positions; {need_rows} needed")
    if workspace is None:
        workspace = new_workspace(need_rows, n_tok, n_heads, n_kv, hd, q.device)
    lib = load_library()
    ws = (_ptr(workspace), workspace.numel() * workspace.element_size())
    if i8:
        _check(lib.gi_attn_decode_i8(_stream(), _ptr(q), q.stride(0), _ptr(k_cache), _ptr(v_cache), _ptr(k_scale),
                                     _ptr(v_scale), kv_stride, kv_head_stride, sc_stride, sc_head_stride, _ptr(out),
                                     out.stride(0), *ws, pos0, _ptr(posp), ctx_cap, n_tok, n_heads, n_kv, hd, scale))
    else:
        _check(lib.gi_attn_decode(_stream(), _ptr(q), q.stride(0), _ptr(k_cache), _ptr(v_cache), kv_stride,
                                  kv_head_stride, _ptr(out), out.stride(0), *ws, pos0, _ptr(posp), ctx_cap, n_tok,
                                  n_heads, n_kv, hd, scale))
    return out


def decode_q4(q, k_cache, v_cache, k_scale, v_scale, pos0, n_heads, n_kv, scale=None, out=None, workspace=None,
              posp=None, ctx_cap=0, kv_layout="reference"):
    """decode over the 4-bit cache (head size 256; attention_decode_tc256 with KV4, src/cuda.rs:2625-2802): q the
    rotated queries f32 [n_tok, >= n_heads*256]; k_cache / v_cache uint8 rows, k_scale / v_scale float16 (see
    _q4_layout). Returns the rotated output f32 [n_tok, n_heads*256] (hadamard_rows turns it back)."""
    _need(q, "q", torch.float32)
    kv_stride, kv_head_stride, sc_stride, sc_head_stride, capacity = _q4_layout(k_cache, v_cache, k_scale, v_scale,
                                                                                n_kv, kv_layout)
    n_tok = q.shape[0]
    if scale is None:
        scale = 1.0 / 16.0
    if out is None:
        out = torch.empty((n_tok, n_heads * 256), dtype=torch.float32, device=q.device)
    _need(out, "out", torch.float32)
    if posp is not None:
        _need(posp, "posp", torch.int32)
    need_rows = ctx_cap if posp is not None else pos0 + n_tok
    if capacity < need_rows:
        raise GiAttnError(f"the cache holds {capacity} positions; {need_rows} needed")
    if workspace is None:
        workspace = new_workspace(need_rows, n_tok, n_heads, n_kv, 256, q.device)
    _check(load_library().gi_attn_decode_q4(_stream(), _ptr(q), q.stride(0), _ptr(k_cache), _ptr(v_cache),
                                            _ptr(k_scale), _ptr(v_scale), kv_stride, kv_head_stride, sc_stride,
                                            sc_head_stride, _ptr(out), out.stride(0), _ptr(workspace),
                                            workspace.numel() * workspace.element_size(), pos0, _ptr(posp), ctx_cap,
                                            n_tok, n_heads, n_kv, scale))
    return out


def prefill_workspace(kv_len, n_kv, hd, fmt, device):
    """A workspace for the pre-widened prefill over kv_len keys (fmt 1 int8, 2 the 4-bit cache), or None where that
    path does not apply (gi_attn_prefill_workspace_bytes is 0)."""
    nbytes = load_library().gi_attn_prefill_workspace_bytes(kv_len, n_kv, hd, fmt)
    return torch.empty(nbytes, dtype=torch.uint8, device=device) if nbytes else None


def prefill_q4(q, k_cache, v_cache, k_scale, v_scale, pos0, n_heads, n_kv, scale=None, out=None, out_dtype=None,
               kv_layout="reference", staged=True, workspace=None):
    """Causal prefill over the 4-bit cache (head size 256; attention_prefill_tc256 with KV4, src/cuda.rs:2495-2514):
    q the rotated queries, f32 or f16 [n, >= n_heads*256]; returns rotated rows of out_dtype (default q's).
    staged: widen the keys into a workspace first (allocated here unless given) and stage the widened tiles as the
    f16 cache's are (the same outputs); else the kernel widens each tile as it stages it."""
    if q.dtype not in (torch.float32, torch.float16):
        raise GiAttnError("q must be float32 or float16")
    _need(q, "q", q.dtype)
    kv_stride, kv_head_stride, sc_stride, sc_head_stride, capacity = _q4_layout(k_cache, v_cache, k_scale, v_scale,
                                                                                n_kv, kv_layout)
    n = q.shape[0]
    if capacity < pos0 + n:
        raise GiAttnError(f"the cache holds {capacity} positions; {pos0 + n} needed")
    if scale is None:
        scale = 1.0 / 16.0
    if out is None:
        out = torch.empty((n, n_heads * 256), dtype=out_dtype or q.dtype, device=q.device)
    if out.dtype not in (torch.float32, torch.float16):
        raise GiAttnError("out must be float32 or float16")
    _need(out, "out", out.dtype)
    qd = GI_F16 if q.dtype == torch.float16 else GI_F32
    od = GI_F16 if out.dtype == torch.float16 else GI_F32
    lib = load_library()
    if staged and workspace is None:
        workspace = prefill_workspace(pos0 + n, n_kv, 256, 2, q.device)
    if staged:
        _need(workspace, "workspace", torch.uint8)
        _check(lib.gi_attn_prefill_q4_ws(_stream(), _ptr(q), qd, q.stride(0), _ptr(k_cache), _ptr(v_cache),
                                         _ptr(k_scale), _ptr(v_scale), kv_stride, kv_head_stride, sc_stride,
                                         sc_head_stride, _ptr(out), od, out.stride(0), pos0, n, n_heads, n_kv, scale,
                                         _ptr(workspace), workspace.numel()))
        return out
    _check(lib.gi_attn_prefill_q4(_stream(), _ptr(q), qd, q.stride(0), _ptr(k_cache), _ptr(v_cache),
                                  _ptr(k_scale), _ptr(v_scale), kv_stride, kv_head_stride, sc_stride,
                                  sc_head_stride, _ptr(out), od, out.stride(0), pos0, n, n_heads, n_kv, scale))
    return out


def attention_q4(qkv, k_cache, v_cache, k_scale, v_scale, pos0, n_heads, n_kv, exact=False, out=None, workspace=None,
                 posp=None, ctx_cap=0):
    """GpuModel::attention over the 4-bit cache (head size 256, the reference layout): qkv rows [q | k | v] f32 with
    the rotated queries qk_norm_rope_q4 leaves; returns the rotated output f32 [n, n_heads*256] (hadamard_rows
    turns it back, as the layer does)."""
    _need(qkv, "qkv", torch.float32)
    n = qkv.shape[0]
    row = (n_heads + 2 * n_kv) * 256
    if qkv.shape[1] != row or not qkv.is_contiguous():
        raise GiAttnError(f"qkv must be contiguous [n, {row}]")
    *_, capacity = _q4_layout(k_cache, v_cache, k_scale, v_scale, n_kv, "reference")
    if capacity < max(pos0 + n, ctx_cap if posp is not None else 0):
        raise GiAttnError(f"the cache holds {capacity} positions; {pos0 + n} needed")
    if out is None:
        out = torch.empty((n, n_heads * 256), dtype=torch.float32, device=qkv.device)
    _need(out, "out", torch.float32)
    if posp is not None:
        _need(posp, "posp", torch.int32)
    ws_ptr, ws_bytes = None, 0
    if n < TILED_MIN_BATCH or exact:
        if workspace is None:
            cap = ctx_cap if posp is not None else pos0 + n
            workspace = new_workspace(cap, min(n, SPLIT_MAX_BATCH), n_heads, n_kv, 256, qkv.device)
        ws_ptr, ws_bytes = _ptr(workspace), workspace.numel() * workspace.element_size()
    else:
        # a prefill batch: the pre-widened staging, whose workspace the library checks
        if workspace is None:
            workspace = prefill_workspace(pos0 + n, n_kv, 256, 2, qkv.device)
        ws_ptr, ws_bytes = _ptr(workspace), workspace.numel() * workspace.element_size()
    _check(load_library().gi_attention_q4(_stream(), _ptr(qkv), _ptr(k_cache), _ptr(v_cache), _ptr(k_scale),
                                          _ptr(v_scale), _ptr(out), ws_ptr, ws_bytes, pos0, _ptr(posp), ctx_cap, n,
                                          n_heads, n_kv, 1 if exact else 0))
    return out


def hadamard_rows(x):
    """hadamard_rows with block 256 (src/cuda.rs:4675-4693), in place on f32 rows [rows, width] (width a multiple of
    256): turns the rotated attention output of a 4-bit cache back."""
    _need(x, "x", torch.float32)
    if x.dim() != 2:
        raise GiAttnError("x must be [rows, width]")
    _check(load_library().gi_hadamard_rows(_stream(), _ptr(x), x.stride(0), x.shape[0], x.shape[1]))
    return x


def prefill(q, k_cache, v_cache, pos0, n_heads, n_kv, hd=128, scale=None, out=None, out_dtype=None,
            kv_layout="reference", k_scale=None, v_scale=None, staged=True, workspace=None, f32=False):
    """Causal prefill of n = q.shape[0] tokens at positions pos0..pos0+n-1 (their K/V already cached).

    q: f32 or f16 [n, >= n_heads*hd]; caches f16, or int8 with f32 k_scale / v_scale; returns
    [n, n_heads*hd] of out_dtype (default: q's dtype). int8 at head sizes 64, 128, 256 with staged: the keys are
    widened into a workspace first (allocated here unless given) and the widened tiles staged as the f16 cache's
    are (the same outputs); else the kernel widens each tile as it stages it. f32: the prompt in f32 (no f16
    rounding of Q or P), the reference's attention_prefill with its tensor-core prefill off (head sizes up to 128).
    """
    if q.dtype not in (torch.float32, torch.float16):
        raise GiAttnError("q must be float32 or float16")
    _need(q, "q", q.dtype)
    kv_stride, kv_head_stride, capacity = _cache_layout(k_cache, v_cache, n_kv, hd, kv_layout,
                                                        (torch.float16, torch.int8))
    i8 = k_cache.dtype == torch.int8
    if i8:
        sc = _scale_layout(k_scale, v_scale, n_kv, capacity, kv_layout)
    n = q.shape[0]
    if capacity < pos0 + n:
        raise GiAttnError(f"the cache holds {capacity} positions; {pos0 + n} needed")
    if scale is None:
        scale = 1.0 / math.sqrt(hd)
    if out is None:
        out = torch.empty((n, n_heads * hd), dtype=out_dtype or q.dtype, device=q.device)
    if out.dtype not in (torch.float32, torch.float16):
        raise GiAttnError("out must be float32 or float16")
    _need(out, "out", out.dtype)
    lib = load_library()
    qd = GI_F16 if q.dtype == torch.float16 else GI_F32
    od = GI_F16 if out.dtype == torch.float16 else GI_F32
    if f32:
        _check(lib.gi_attn_prefill_f32(_stream(), _ptr(q), qd, q.stride(0), _ptr(k_cache), _ptr(v_cache),
                                       _ptr(k_scale) if i8 else None, _ptr(v_scale) if i8 else None, 1 if i8 else 0,
                                       kv_stride, kv_head_stride, sc[0] if i8 else 0, sc[1] if i8 else 0, _ptr(out), od,
                                       out.stride(0), pos0, n, n_heads, n_kv, hd, scale))
    elif i8 and staged and hd in (64, 128, 256):
        if workspace is None:
            workspace = prefill_workspace(pos0 + n, n_kv, hd, 1, q.device)
        _need(workspace, "workspace", torch.uint8)
        _check(lib.gi_attn_prefill_i8_ws(_stream(), _ptr(q), qd, q.stride(0), _ptr(k_cache), _ptr(v_cache),
                                         _ptr(k_scale), _ptr(v_scale), kv_stride, kv_head_stride, sc[0], sc[1],
                                         _ptr(out), od, out.stride(0), pos0, n, n_heads, n_kv, hd, scale,
                                         _ptr(workspace), workspace.numel()))
    elif i8:
        _check(lib.gi_attn_prefill_i8(_stream(), _ptr(q), qd, q.stride(0), _ptr(k_cache), _ptr(v_cache), _ptr(k_scale),
                                      _ptr(v_scale), kv_stride, kv_head_stride, sc[0], sc[1], _ptr(out), od,
                                      out.stride(0), pos0, n, n_heads, n_kv, hd, scale))
    else:
        _check(lib.gi_attn_prefill(_stream(), _ptr(q), qd, q.stride(0), _ptr(k_cache), _ptr(v_cache), kv_stride,
                                   kv_head_stride, _ptr(out), od, out.stride(0), pos0, n, n_heads, n_kv, hd, scale))
    return out


def attention(qkv, k_cache, v_cache, pos0, n_heads, n_kv, hd=128, exact=False, out=None, workspace=None,
              posp=None, ctx_cap=0, k_scale=None, v_scale=None, no_tc=False):
    """GpuModel::attention (src/cuda.rs:8448-8541) for one layer.

    qkv: f32 [n, n_heads*hd + 2*n_kv*hd] rows [q | k | v] (only q is read: the cache already holds this
    batch's K/V rows, as qk_norm_rope wrote them); returns f32 [n, n_heads*hd]. n >= 16 and not exact ->
    causal prefill kernel; otherwise the split decode path, 15 tokens per launch. The caches are the
    reference's [capacity, n_kv, hd]: f16, or int8 with f32 scales [capacity, n_kv] (its (kc, vc, ks, vs)).
    no_tc: the reference's GHOST_INFER_NO_TC_ATT: batches of >= 16 tokens in f32 (head sizes up to 128; above, the
    split path), and at head size 256 over the int8 cache the split path in f32 precision instead of the tc256
    roundings.
    """
    _need(qkv, "qkv", torch.float32)
    n = qkv.shape[0]
    row = n_heads * hd + 2 * n_kv * hd
    if qkv.shape[1] != row or not qkv.is_contiguous():
        raise GiAttnError(f"qkv must be contiguous [n, {row}]")
    _, _, capacity = _cache_layout(k_cache, v_cache, n_kv, hd, "reference", (torch.float16, torch.int8))
    i8 = k_cache.dtype == torch.int8
    if i8:
        _scale_layout(k_scale, v_scale, n_kv, capacity, "reference")
    if capacity < max(pos0 + n, ctx_cap if posp is not None else 0):
        raise GiAttnError(f"the cache holds {capacity} positions; {pos0 + n} needed")
    if out is None:
        out = torch.empty((n, n_heads * hd), dtype=torch.float32, device=qkv.device)
    _need(out, "out", torch.float32)
    if posp is not None:
        _need(posp, "posp", torch.int32)
    ws_ptr, ws_bytes = None, 0
    code = (1 if exact else 0) | (2 if no_tc else 0)  # the library's exact bits: verify, no tensor-core kernels
    split = n < TILED_MIN_BATCH or exact or (no_tc and hd > 128)
    if split:
        if workspace is None:
            cap = ctx_cap if posp is not None else pos0 + n
            workspace = new_workspace(cap, min(n, SPLIT_MAX_BATCH), n_heads, n_kv, hd, qkv.device)
        ws_ptr, ws_bytes = _ptr(workspace), workspace.numel() * workspace.element_size()
    elif i8 and not no_tc:
        # a prefill batch over the int8 cache: the pre-widened staging, whose workspace the library checks
        if workspace is None:
            workspace = prefill_workspace(pos0 + n, n_kv, hd, 1, qkv.device)
        if workspace is not None:
            ws_ptr, ws_bytes = _ptr(workspace), workspace.numel() * workspace.element_size()
    lib = load_library()
    if i8:
        _check(lib.gi_attention_i8(_stream(), _ptr(qkv), _ptr(k_cache), _ptr(v_cache), _ptr(k_scale), _ptr(v_scale),
                                   _ptr(out), ws_ptr, ws_bytes, pos0, _ptr(posp), ctx_cap, n, n_heads, n_kv, hd, code))
    else:
        _check(lib.gi_attention(_stream(), _ptr(qkv), _ptr(k_cache), _ptr(v_cache), _ptr(out), ws_ptr, ws_bytes, pos0,
                                _ptr(posp), ctx_cap, n, n_heads, n_kv, hd, code))
    return out


def qk_norm_rope(qkv, k_cache, v_cache, pos0, n_heads, n_kv, hd=128, rope_dim=None, base=10000.0, qn=None, kn=None,
                 ff=None, neox=True, eps=1e-6, posp=None, kv_layout="reference", k_scale=None, v_scale=None,
                 ctx_cap=None):
    """RMSNorm + RoPE of the q and k heads of f32 rows [q | k | v] (in place) and the k and v heads into the
    caches at positions pos0.. (layer_attn's qk_norm_rope step, src/cuda.rs:437-486): f16 caches, or int8
    ones quantised per row into k_scale / v_scale (kv_store with KV8, src/cuda.rs:333-339). Rows at positions
    past ctx_cap (default: the cache's capacity) are not stored, so a device position cannot write past it."""
    _need(qkv, "qkv", torch.float32)
    if not qkv.is_contiguous() or qkv.dim() != 2 or qkv.shape[1] != (n_heads + 2 * n_kv) * hd:
        raise GiAttnError(f"qkv must be contiguous [n, {(n_heads + 2 * n_kv) * hd}]")
    kv_stride, kv_head_stride, capacity = _cache_layout(k_cache, v_cache, n_kv, hd, kv_layout,
                                                        (torch.float16, torch.int8))
    n = qkv.shape[0]
    if posp is None and capacity < pos0 + n:
        raise GiAttnError(f"the cache holds {capacity} positions; {pos0 + n} needed")
    for t, name in ((qn, "qn"), (kn, "kn"), (ff, "ff")):
        if t is not None:
            _need(t, name, torch.float32)
    if posp is not None:
        _need(posp, "posp", torch.int32)
    cap = capacity if ctx_cap is None else ctx_cap
    if cap > capacity:
        raise GiAttnError(f"ctx_cap {cap} exceeds the cache's {capacity} positions")
    rope = (hd if rope_dim is None else rope_dim, base, _ptr(ff), 1 if neox else 0, eps)
    if k_cache.dtype == torch.int8:
        sc_stride, sc_head_stride = _scale_layout(k_scale, v_scale, n_kv, capacity, kv_layout)
        _check(load_library().gi_qk_norm_rope_i8(_stream(), _ptr(qkv), _ptr(qn), _ptr(kn), _ptr(k_cache),
                                                 _ptr(v_cache), _ptr(k_scale), _ptr(v_scale), kv_stride,
                                                 kv_head_stride, sc_stride, sc_head_stride, pos0, _ptr(posp), cap,
                                                 n, n_heads, n_kv, hd, *rope))
    else:
        _check(load_library().gi_qk_norm_rope(_stream(), _ptr(qkv), _ptr(qn), _ptr(kn), _ptr(k_cache), _ptr(v_cache),
                                              kv_stride, kv_head_stride, pos0, _ptr(posp), cap, n, n_heads, n_kv,
                                              hd, *rope))
    return qkv


def qk_norm_rope_q4(qkv, k_cache, v_cache, k_scale, v_scale, pos0, n_heads, n_kv, rope_dim=None, base=10000.0,
                    qn=None, kn=None, ff=None, neox=True, eps=1e-6, posp=None, kv_layout="reference", ctx_cap=None):
    """qk_norm_rope into the 4-bit cache (head size 256; qk_norm_rope with KV4, src/cuda.rs:437-486, 340-357): q
    and k heads rotated after RoPE (in place), k rows quantised, v rows rotated and quantised."""
    _need(qkv, "qkv", torch.float32)
    if not qkv.is_contiguous() or qkv.dim() != 2 or qkv.shape[1] != (n_heads + 2 * n_kv) * 256:
        raise GiAttnError(f"qkv must be contiguous [n, {(n_heads + 2 * n_kv) * 256}]")
    kv_stride, kv_head_stride, sc_stride, sc_head_stride, capacity = _q4_layout(k_cache, v_cache, k_scale, v_scale,
                                                                                n_kv, kv_layout)
    n = qkv.shape[0]
    if posp is None and capacity < pos0 + n:
        raise GiAttnError(f"the cache holds {capacity} positions; {pos0 + n} needed")
    for t, name in ((qn, "qn"), (kn, "kn"), (ff, "ff")):
        if t is not None:
            _need(t, name, torch.float32)
    if posp is not None:
        _need(posp, "posp", torch.int32)
    cap = capacity if ctx_cap is None else ctx_cap
    if cap > capacity:
        raise GiAttnError(f"ctx_cap {cap} exceeds the cache's {capacity} positions")
    _check(load_library().gi_qk_norm_rope_q4(_stream(), _ptr(qkv), _ptr(qn), _ptr(kn), _ptr(k_cache), _ptr(v_cache),
                                             _ptr(k_scale), _ptr(v_scale), kv_stride, kv_head_stride, sc_stride,
                                             sc_head_stride, pos0, _ptr(posp), cap, n, n_heads, n_kv,
                                             256 if rope_dim is None else rope_dim, base, _ptr(ff), 1 if neox else 0,
                                             eps))
    return qkv


def kv_relayout(src, dst, n_rows, layout="head_major", n_kv=None):
    """Cache growth (LayerCache::resize's copy of the first n_rows positions, src/cuda.rs:9962-9976): copies
    positions 0..n_rows-1 of every kv head from cache `src` into `dst` of a larger capacity, in the same
    layout. head_major: [n_kv, cap, row...] (every row moves); reference: [cap, n_kv, row...] (or [cap, n_kv]
    scales). Works for f16 and int8 rows and f32 scales; returns dst."""
    if src.dtype != dst.dtype or not src.is_contiguous() or not dst.is_contiguous():
        raise GiAttnError("src and dst must be contiguous tensors of one dtype")
    _need(src, "src", src.dtype)
    _need(dst, "dst", dst.dtype)
    es = src.element_size()
    if layout == "head_major":
        if src.dim() < 2 or src.shape[0] != dst.shape[0] or src.shape[2:] != dst.shape[2:]:
            raise GiAttnError("head-major caches must be [n_kv, cap, ...] with equal rows")
        n_kv = src.shape[0]
        row = es * (src[0, 0].numel())
        cap_s, cap_d = src.shape[1], dst.shape[1]
        strides = (row, cap_s * row, row, cap_d * row)
    elif layout == "reference":
        if src.dim() < 2 or src.shape[1:] != dst.shape[1:]:
            raise GiAttnError("reference caches must be [cap, n_kv, ...] with equal rows")
        n_kv = src.shape[1]
        row = es * (src[0, 0].numel())
        cap_s, cap_d = src.shape[0], dst.shape[0]
        strides = (n_kv * row, row, n_kv * row, row)
    else:
        raise GiAttnError(f"unknown cache layout {layout!r}")
    if n_rows > min(cap_s, cap_d):
        raise GiAttnError(f"{n_rows} rows do not fit capacities {cap_s} and {cap_d}")
    _check(load_library().gi_kv_relayout(_stream(), _ptr(src), strides[0], strides[1], _ptr(dst), strides[2],
                                         strides[3], n_rows, n_kv, row))
    return dst


def kernel_timing(on):
    """Switches per-kernel event timing on or off (benchmarks only; launches under graph capture are
    not timed)."""
    _check(load_library().gi_kernel_timing(1 if on else 0))


def kernel_timing_read(kernel):
    """(total milliseconds, launches) of kernel kind "decode_partial", "decode_combine", "prefill",
    "qk_norm_rope", "kv_relayout", "hadamard_rows" or "kv_widen" since the previous read of that kind."""
    ms, n = ctypes.c_double(), ctypes.c_int()
    _check(load_library().gi_kernel_timing_read(kernel.encode(), ctypes.byref(ms), ctypes.byref(n)))
    return ms.value, n.value
