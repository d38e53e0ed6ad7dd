"""ctypes wrapper of the CPU oracle (oracle/_build/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py as the checker.  The product library never uses it.
Arrays are numpy uint16 (fp16 bit patterns) or float32.
"""
from __future__ import annotations

import ctypes
import pathlib
import subprocess

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
LIB = HERE / "_build" / "liboracle.so"

_lib = None
_vp = ctypes.c_void_p
_sz = ctypes.c_size_t


def build():
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


def lib():
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        L = ctypes.CDLL(str(LIB))
        L.orc_f32_to_f16.restype = ctypes.c_uint16
        L.orc_f32_to_f16.argtypes = [ctypes.c_float]
        L.orc_f16_to_f32.restype = ctypes.c_float
        L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_f32_to_f16_array.argtypes = [_vp, _vp, _sz]
        L.orc_f16_to_f32_array.argtypes = [_vp, _vp, _sz]
        L.orc_rope_tables.argtypes = [_vp, _vp, _sz, _sz, ctypes.c_float]
        L.orc_rope_store_kv.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz,
                                        _sz, _sz, _sz, ctypes.c_int]
        L.orc_attention.restype = ctypes.c_int
        L.orc_attention.argtypes = [_vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _sz, _sz, _sz,
                                    _sz, ctypes.c_int, _vp, _sz]
        L.orc_attention_chunked.restype = ctypes.c_int
        L.orc_attention_chunked.argtypes = [_vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _sz, _sz]
        for f in ("orc_kv_k_offset", "orc_kv_v_offset"):
            getattr(L, f).restype = _sz
            getattr(L, f).argtypes = [_sz, _sz, _sz, _sz]
        L.orc_kv_total_bytes.restype = _sz
        L.orc_kv_total_bytes.argtypes = [_sz, _sz, _sz, _sz]
        L.orc_kat_inputs.argtypes = [_vp, _vp, _vp, _sz, _sz, _sz, _sz]
        L.orc_gemv.argtypes = [_vp, _vp, _vp, _sz, _sz]
        L.orc_gemm.argtypes = [_vp, _vp, _vp, _sz, _sz, _sz]
        L.orc_gemv_beta.argtypes = [_vp, _vp, _vp, _sz, _sz, ctypes.c_float]
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data


def f32_to_f16(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().orc_f32_to_f16_array(_p(x), _p(out), x.size)
    return out


def f16_to_f32(h) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib().orc_f16_to_f32_array(_p(h), _p(out), h.size)
    return out


def rope_tables(max_seq_len, head_dim, theta):
    half = head_dim // 2
    c = np.empty((max_seq_len, half), dtype=np.uint16)
    s = np.empty((max_seq_len, half), dtype=np.uint16)
    lib().orc_rope_tables(_p(c), _p(s), max_seq_len, head_dim, float(theta))
    return c, s


def rope_store_kv(q, k, v, k_cache, v_cache, cos, sin, seq_len, num_heads, num_kv_heads,
                  head_dim, q_stride, k_stride, start_pos, apply_rotation):
    """In-place on q (and k when k_cache is None), k_cache, v_cache (uint16 arrays)."""
    for a in (q, k, v, k_cache, v_cache, cos, sin):
        assert a is None or (a.dtype == np.uint16 and a.flags.c_contiguous)
    lib().orc_rope_store_kv(_p(q), _p(k), _p(v), _p(k_cache), _p(v_cache), _p(cos), _p(sin),
                            seq_len, num_heads, num_kv_heads, head_dim, q_stride, k_stride,
                            start_pos, 1 if apply_rotation else 0)


def attention(q, k, v, nq, num_heads, num_kv_heads, head_dim, q_stride, kv_stride, kv_len,
              q_pos0=0, causal=True, rows=None):
    """fp64-softmax GQA attention.  Returns (out16 uint16, out32 float32), each
    [len(rows) or nq, num_heads, head_dim]."""
    cnt = nq if rows is None else len(rows)
    out16 = np.empty((cnt, num_heads, head_dim), dtype=np.uint16)
    out32 = np.empty((cnt, num_heads, head_dim), dtype=np.float32)
    r = None if rows is None else np.ascontiguousarray(rows, dtype=np.int64)
    rc = lib().orc_attention(_p(q), _p(k), _p(v), _p(out16), _p(out32), nq, num_heads,
                             num_kv_heads, head_dim, q_stride, kv_stride, kv_len, q_pos0,
                             1 if causal else 0, _p(r), 0 if r is None else len(r))
    assert rc == 0
    return out16, out32


def attention_chunked(q, k, v, num_heads, num_kv_heads, head_dim, kv_stride, kv_len, chunk):
    out = np.empty((num_heads, head_dim), dtype=np.float32)
    rc = lib().orc_attention_chunked(_p(q), _p(k), _p(v), _p(out), num_heads, num_kv_heads,
                                     head_dim, kv_stride, kv_len, chunk)
    assert rc == 0
    return out


def kv_offsets(layer, max_seq_len, num_kv_heads, head_dim):
    L = lib()
    return (L.orc_kv_k_offset(layer, max_seq_len, num_kv_heads, head_dim),
            L.orc_kv_v_offset(layer, max_seq_len, num_kv_heads, head_dim))


def kv_total_bytes(num_layers, max_seq_len, num_kv_heads, head_dim):
    return lib().orc_kv_total_bytes(num_layers, max_seq_len, num_kv_heads, head_dim)


def kat_inputs(heads, head_dim, kv_heads, length, stride):
    """The reference Flash-Decode known-answer inputs (test_causal_attention.cpp:165-175)."""
    q_dim = heads * head_dim
    kv_dim = kv_heads * head_dim
    q = np.empty(q_dim, dtype=np.uint16)
    k = np.empty((length + 2) * stride, dtype=np.uint16)
    v = np.empty((length + 2) * stride, dtype=np.uint16)
    lib().orc_kat_inputs(_p(q), _p(k), _p(v), q_dim, length, kv_dim, stride)
    return q, k, v


def gemv(w, x):
    """y = fp16(W x) with an fp64 sum (attn_oracle.c:orc_gemv); w uint16 [out][in]."""
    w = np.ascontiguousarray(w, dtype=np.uint16)
    x = np.ascontiguousarray(x, dtype=np.uint16)
    out_dim, in_dim = w.shape
    assert x.shape == (in_dim,)
    y = np.empty(out_dim, dtype=np.uint16)
    lib().orc_gemv(_p(w), _p(x), _p(y), out_dim, in_dim)
    return y


def gemv_beta(w, x, y, beta):
    """fp16(W x + beta y) with an fp64 sum rounded to fp32, then the fp32
    residual add (attn_oracle.c:orc_gemv_beta); returns the new y."""
    w = np.ascontiguousarray(w, dtype=np.uint16)
    x = np.ascontiguousarray(x, dtype=np.uint16)
    out_dim, in_dim = w.shape
    assert x.shape == (in_dim,)
    out = np.array(y, dtype=np.uint16, copy=True)
    assert out.shape == (out_dim,)
    lib().orc_gemv_beta(_p(w), _p(x), _p(out), out_dim, in_dim, float(beta))
    return out


def gemm(x, w):
    """y[m] = fp16(W x[m]) with fp64 sums (attn_oracle.c:orc_gemm); x uint16
    [rows][in], w uint16 [out][in]."""
    x = np.ascontiguousarray(x, dtype=np.uint16)
    w = np.ascontiguousarray(w, dtype=np.uint16)
    rows, in_dim = x.shape
    out_dim = w.shape[0]
    assert w.shape == (out_dim, in_dim)
    y = np.empty((rows, out_dim), dtype=np.uint16)
    lib().orc_gemm(_p(x), _p(w), _p(y), rows, out_dim, in_dim)
    return y


def qkv_rope_store_kv_decode(w, x, k_cache, v_cache, cos, sin, num_heads, num_kv_heads,
                             head_dim, start_pos, apply_rotation):
    """One decode step of model_inference.hpp:354-369: the QKV GEMV, then
    rope_store_kv on its output (Q rotated in place, K rotated into the cache,
    V copied).  Returns y; updates the caches in place."""
    y = gemv(w, x)
    q_dim, kv_dim = num_heads * head_dim, num_kv_heads * head_dim
    q = y[:q_dim].copy()
    k = y[q_dim:q_dim + kv_dim].copy()
    v = y[q_dim + kv_dim:].copy()
    rope_store_kv(q, k, v, k_cache, v_cache, cos, sin, 1, num_heads, num_kv_heads, head_dim,
                  q_dim, kv_dim, start_pos, apply_rotation)
    y[:q_dim] = q
    return y
