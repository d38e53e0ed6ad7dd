"""Python harness for libattn_mi355x.so (the MI355X attention hot path).

This module is a thin ctypes binding of the C ABI declared in
include/attn_mi355x.h.  It mirrors the reference's launch API
(include/kernels/kernels.hpp of MarcVivas/llm-inference): same argument
names, meanings and no-op rules.  Device memory and streams come from
PyTorch (plumbing only); every computation runs in the HIP kernels of the
library.  There is no CPU fallback: if the library is missing, loading fails
loudly.

torch is imported before the library is loaded so that both bind the same HIP
runtime (both are linked against SONAME libamdhip64.so.7).
"""
from __future__ import annotations

import ctypes
import math
import pathlib
from typing import Optional

import torch  # noqa: F401  (must precede the CDLL load, see module docstring)

PKG_ROOT = pathlib.Path(__file__).resolve().parents[2]
LIB_PATH = PKG_ROOT / "lib" / "libattn_mi355x.so"
KV_CHUNK = 12  # kernels.hpp:103

_lib = None

_c = ctypes
_vp = _c.c_void_p
_sz = _c.c_size_t


class AttnError(RuntimeError):
    pass


class ModelConfigC(ctypes.Structure):
    """attn_model_config: the 44-byte weights.bin header (model_config.hpp:10-24)."""
    _fields_ = [("magic", _c.c_char * 4)] + [
        (f, _c.c_uint32) for f in ("vocab_size", "hidden_size", "num_layers", "num_heads",
                                   "num_kv_heads", "head_dim", "intermediate_size",
                                   "max_seq_len")] + [
        ("rms_norm_eps", _c.c_float), ("rope_theta", _c.c_float)]


WEIGHT_LAYER_FIELDS = ("input_norm", "q_proj", "k_proj", "v_proj", "q_norm", "k_norm", "o_proj",
                       "post_attn_norm", "gate_proj", "up_proj", "down_proj")


class WeightsLayout(ctypes.Structure):
    """attn_weights_layout (include/attn_mi355x.h)."""
    _fields_ = [("config", ModelConfigC), ("has_qk_norm", _c.c_uint32)] + [
        (f, _c.c_uint64) for f in ("tokenizer_offset", "tokenizer_bytes", "weights_offset",
                                   "weights_bytes", "layout_bytes", "embedding", "final_norm",
                                   "lm_head", "layer_base", "layer_elems")] + [
        (f, _c.c_uint64) for f in WEIGHT_LAYER_FIELDS]


def _declare(lib):
    sig = {
        "attn_rope_store_kv": (_c.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz,
                                          _sz, _sz, _sz, _c.c_int, _vp]),
        "attn_rope": (_c.c_int, [_vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _sz, _sz, _sz, _vp]),
        "attn_update_rope_node": (_c.c_int, [_vp, _vp, _sz, _c.c_int]),
        "attn_prefill": (_c.c_int, [_vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _sz, _sz, _vp]),
        "attn_decode": (_c.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _sz,
                                   _sz, _sz, _sz, _vp, _vp, _vp]),
        "attn_update_decode_node": (_c.c_int, [_vp, _vp, _sz]),
        "attn_update_merge_node": (_c.c_int, [_vp, _vp, _sz]),
        "attn_decode_workspace_states": (_sz, [_sz, _sz]),
        "attn_rope_tables": (_c.c_int, [_vp, _vp, _sz, _sz, _c.c_float]),
        "attn_decode_plan": (_c.c_int, [_sz, _sz, _sz, _sz, _sz, _vp, _vp, _vp,
                                        _c.POINTER(_c.c_uint32)]),
        "attn_prefill_plan": (_c.c_int, [_vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _sz]),
        "attn_set_option": (_c.c_int, [_c.c_char_p, _c.c_long]),
        "attn_version": (_c.c_char_p, []),
        "attn_qkv_decode": (_c.c_int, [_vp, _vp, _vp, _sz, _sz, _vp]),
        "attn_qkv_rope_store_kv_decode": (_c.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz,
                                                     _sz, _sz, _sz, _sz, _c.c_int, _vp]),
        "attn_update_qkv_rope_node": (_c.c_int, [_vp, _vp, _sz, _c.c_int]),
        "attn_qkv_gemm": (_c.c_int, [_vp, _vp, _vp, _sz, _sz, _sz, _vp]),
        "attn_qkv_gemm_rope_store_kv": (_c.c_int, [_vp] * 7 + [_sz] * 6 + [_c.c_int, _vp]),
        "attn_rope_store_kv_decode": (_c.c_int, [_vp] * 11 + [_sz] * 6 + [_c.c_int, _vp, _vp,
                                                                          _vp]),
        "attn_update_rope_decode_nodes": (_c.c_int, [_vp, _vp, _vp, _sz, _sz, _c.c_int]),
        "attn_decode_noalloc": (_c.c_int, [_vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _sz, _vp]),
        "attn_out_proj_decode": (_c.c_int, [_vp, _vp, _vp, _sz, _sz, _sz, _c.c_float, _vp]),
        "attn_decode_out_proj_workspace_bytes": (_sz, [_sz, _sz]),
        "attn_decode_out_proj": (_c.c_int, [_vp] * 7 + [_sz] * 5 + [_vp, _vp, _sz, _c.c_float,
                                                                    _vp, _vp, _vp, _vp]),
        "attn_weights_parse": (_c.c_int, [_vp, _sz, _c.c_uint64, _c.POINTER(WeightsLayout)]),
        "attn_weights_layout_for": (_c.c_int, [_c.POINTER(ModelConfigC), _c.c_uint64,
                                               _c.POINTER(WeightsLayout)]),
        "attn_weights_error_string": (_c.c_char_p, [_c.c_int]),
        "attn_graph_node_records": (_sz, []),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def lib():
    """Load (once) and return the ctypes handle of libattn_mi355x.so."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise AttnError(f"{LIB_PATH} is not built: run `python -c 'import __graft_entry__ as g; g.build()'`")
        _lib = _declare(ctypes.CDLL(str(LIB_PATH)))
    return _lib


def exported_symbols():
    """Names declared in include/attn_mi355x.h."""
    return ["attn_rope_store_kv", "attn_rope", "attn_update_rope_node", "attn_prefill",
            "attn_decode", "attn_update_decode_node", "attn_update_merge_node",
            "attn_decode_workspace_states", "attn_rope_tables", "attn_decode_plan",
            "attn_prefill_plan", "attn_set_option", "attn_version", "attn_qkv_decode",
            "attn_qkv_rope_store_kv_decode", "attn_update_qkv_rope_node", "attn_qkv_gemm",
            "attn_qkv_gemm_rope_store_kv", "attn_rope_store_kv_decode",
            "attn_update_rope_decode_nodes", "attn_weights_parse", "attn_weights_layout_for",
            "attn_decode_noalloc", "attn_out_proj_decode",
            "attn_decode_out_proj_workspace_bytes", "attn_decode_out_proj",
            "attn_weights_error_string", "attn_graph_node_records"]


def _ptr(x) -> Optional[int]:
    if x is None:
        return None
    if isinstance(x, int):
        return x
    return x.data_ptr()


def _stream(stream) -> Optional[int]:
    if stream is None:
        return torch.cuda.current_stream().cuda_stream
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream


def _check(rc: int, what: str):
    if rc != 0:
        raise AttnError(f"{what} failed with hipError {rc}")


def set_option(name: str, value: int):
    if lib().attn_set_option(name.encode(), int(value)) != 0:
        raise AttnError(f"unknown option {name}")


def decode_workspace_states(num_heads: int, kv_len: int) -> int:
    return int(lib().attn_decode_workspace_states(num_heads, kv_len))


def rope_tables(max_seq_len: int, head_dim: int, rope_theta: float):
    """Host fp16 cos/sin tables [max_seq_len, head_dim/2] (rope_cache.hpp:48-76),
    returned as CPU int16 tensors holding fp16 bits viewed as float16."""
    half = head_dim // 2
    cos = torch.empty(max_seq_len * half, dtype=torch.float16)
    sin = torch.empty(max_seq_len * half, dtype=torch.float16)
    _check(lib().attn_rope_tables(cos.data_ptr(), sin.data_ptr(), max_seq_len, head_dim,
                                  float(rope_theta)), "attn_rope_tables")
    return cos.view(max_seq_len, half), sin.view(max_seq_len, half)


def rope_store_kv(q, k, v, k_cache, v_cache, cos, sin, seq_len, num_heads, num_kv_heads,
                  head_dim, q_stride, k_stride, start_pos, apply_rotation, stream=None):
    """launch_rope_and_store_kv (kernels.hpp:62-79).  Tensor or int pointers."""
    rc = lib().attn_rope_store_kv(_ptr(q), _ptr(k), _ptr(v), _ptr(k_cache), _ptr(v_cache),
                                  _ptr(cos), _ptr(sin), seq_len, num_heads, num_kv_heads,
                                  head_dim, q_stride, k_stride, start_pos,
                                  1 if apply_rotation else 0, _stream(stream))
    _check(rc, "attn_rope_store_kv")


def qkv_decode(x, y, w, hidden_size, total_qkv_dim, stream=None):
    """launch_qkv_decode (kernels.hpp:38-45): y = W x, fp16 out."""
    rc = lib().attn_qkv_decode(_ptr(x), _ptr(y), _ptr(w), hidden_size, total_qkv_dim,
                               _stream(stream))
    _check(rc, "attn_qkv_decode")


def qkv_rope_store_kv_decode(x, y, w, k_cache, v_cache, cos, sin, hidden_size, num_heads,
                             num_kv_heads, head_dim, start_pos, apply_rotation, stream=None):
    """launch_qkv_decode + launch_rope_and_store_kv of one decode step, fused."""
    rc = lib().attn_qkv_rope_store_kv_decode(_ptr(x), _ptr(y), _ptr(w), _ptr(k_cache),
                                             _ptr(v_cache), _ptr(cos), _ptr(sin), hidden_size,
                                             num_heads, num_kv_heads, head_dim, start_pos,
                                             1 if apply_rotation else 0, _stream(stream))
    _check(rc, "attn_qkv_rope_store_kv_decode")


def qkv_gemm(x, y, w, seq_len, hidden_size, total_qkv_dim, stream=None):
    """launch_qkv_gemm (kernels.hpp:29-36): y[seq][total] = x[seq][hidden] . W^T."""
    rc = lib().attn_qkv_gemm(_ptr(x), _ptr(y), _ptr(w), seq_len, hidden_size, total_qkv_dim,
                             _stream(stream))
    _check(rc, "attn_qkv_gemm")


def qkv_gemm_rope_store_kv(x, y, w, k_cache, v_cache, cos, sin, seq_len, hidden_size, num_heads,
                           num_kv_heads, head_dim, start_pos, apply_rotation, stream=None):
    """launch_qkv_gemm + launch_rope_and_store_kv of a prefill, fused."""
    rc = lib().attn_qkv_gemm_rope_store_kv(_ptr(x), _ptr(y), _ptr(w), _ptr(k_cache),
                                           _ptr(v_cache), _ptr(cos), _ptr(sin), seq_len,
                                           hidden_size, num_heads, num_kv_heads, head_dim,
                                           start_pos, 1 if apply_rotation else 0,
                                           _stream(stream))
    _check(rc, "attn_qkv_gemm_rope_store_kv")


def rope(q, k, cos, sin, seq_len, num_heads, num_kv_heads, head_dim, q_stride, k_stride,
         start_pos=0, stream=None):
    """launch_rope (kernels.hpp:47-59)."""
    rc = lib().attn_rope(_ptr(q), _ptr(k), _ptr(cos), _ptr(sin), seq_len, num_heads,
                         num_kv_heads, head_dim, q_stride, k_stride, start_pos, _stream(stream))
    _check(rc, "attn_rope")


def prefill(q, k, v, out, seq_len, num_heads, num_kv_heads, head_dim, q_stride=0,
            kv_stride=0, stream=None):
    """launch_causal_attention_prefill (kernels.hpp:88-99)."""
    rc = lib().attn_prefill(_ptr(q), _ptr(k), _ptr(v), _ptr(out), seq_len, num_heads,
                            num_kv_heads, head_dim, q_stride, kv_stride, _stream(stream))
    _check(rc, "attn_prefill")


def decode(q, k_cache, v_cache, out, partial_out, partial_max, partial_sum, query_len,
           kv_len, start_pos, num_heads, num_kv_heads, head_dim, q_stride=0, kv_stride=0,
           stream=None):
    """launch_causal_attention_decode[_vectorized] (kernels.hpp:104-146)."""
    rc = lib().attn_decode(_ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(out),
                           _ptr(partial_out), _ptr(partial_max), _ptr(partial_sum), query_len,
                           kv_len, start_pos, num_heads, num_kv_heads, head_dim, q_stride,
                           kv_stride, _stream(stream), None, None)
    _check(rc, "attn_decode")


def rope_store_kv_decode(q, k, v, k_cache, v_cache, cos, sin, out, partial_out, partial_max,
                         partial_sum, kv_len, start_pos, num_heads, num_kv_heads, head_dim,
                         apply_rotation=True, kv_stride=0, stream=None, nodes=None):
    """launch_rope_and_store_kv + launch_causal_attention_decode for one decode
    token as the decode's two kernels (no reference counterpart).  `nodes`, a
    list, receives the (split, merge) graph nodes when capturing."""
    an, mn = ctypes.c_void_p(), ctypes.c_void_p()
    rc = lib().attn_rope_store_kv_decode(
        _ptr(q), _ptr(k), _ptr(v), _ptr(k_cache), _ptr(v_cache), _ptr(cos), _ptr(sin), _ptr(out),
        _ptr(partial_out), _ptr(partial_max), _ptr(partial_sum), kv_len, start_pos, num_heads,
        num_kv_heads, head_dim, kv_stride, 1 if apply_rotation else 0, _stream(stream),
        ctypes.byref(an) if nodes is not None else None,
        ctypes.byref(mn) if nodes is not None else None)
    _check(rc, "attn_rope_store_kv_decode")
    if nodes is not None:
        nodes[:] = [an.value, mn.value]


def update_rope_decode_nodes(graph_exec, attention_node, merge_node, kv_len, start_pos,
                             apply_rotation=True):
    rc = lib().attn_update_rope_decode_nodes(graph_exec, attention_node, merge_node, kv_len,
                                             start_pos, 1 if apply_rotation else 0)
    _check(rc, "attn_update_rope_decode_nodes")


def out_proj_decode(x, y, w, hidden_size, num_heads, head_dim, beta, stream=None):
    """launch_attention_out_projection_decode (kernels.hpp:179-187):
    y = W x + beta y, fp16 out."""
    rc = lib().attn_out_proj_decode(_ptr(x), _ptr(y), _ptr(w), hidden_size, num_heads,
                                    head_dim, float(beta), _stream(stream))
    _check(rc, "attn_out_proj_decode")


def decode_out_proj_workspace(num_heads: int, hidden_size: int, device="cuda"):
    """The zero-filled workspace attn_decode_out_proj needs (fp32 head partials
    and per-row-block counters; every call leaves the counters zero)."""
    n = int(lib().attn_decode_out_proj_workspace_bytes(num_heads, hidden_size))
    return torch.zeros(n, dtype=torch.uint8, device=device)


def decode_out_proj(q, k_cache, v_cache, attn_out, partial_out, partial_max, partial_sum,
                    kv_len, num_heads, num_kv_heads, head_dim, w_o, y, hidden_size, beta,
                    workspace, kv_stride=0, stream=None, nodes=None):
    """launch_causal_attention_decode + launch_attention_out_projection_decode
    of one decode step with the merge and the projection in one kernel (no
    reference counterpart).  `nodes`, a list, receives the (split, merge)
    graph nodes when capturing."""
    an, mn = ctypes.c_void_p(), ctypes.c_void_p()
    rc = lib().attn_decode_out_proj(
        _ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(attn_out), _ptr(partial_out),
        _ptr(partial_max), _ptr(partial_sum), kv_len, num_heads, num_kv_heads, head_dim,
        kv_stride, _ptr(w_o), _ptr(y), hidden_size, float(beta), _ptr(workspace),
        _stream(stream), ctypes.byref(an) if nodes is not None else None,
        ctypes.byref(mn) if nodes is not None else None)
    _check(rc, "attn_decode_out_proj")
    if nodes is not None:
        nodes[:] = [an.value, mn.value]


def decode_plan(kv_len, num_heads, num_kv_heads, head_dim, kv_stride=0, q=None, k=None,
                v=None):
    out = (ctypes.c_uint32 * 5)()
    rc = lib().attn_decode_plan(kv_len, num_heads, num_kv_heads, head_dim, kv_stride,
                                _ptr(q) or 256, _ptr(k) or 256, _ptr(v) or 256, out)
    _check(rc, "attn_decode_plan")
    return {"path": out[0], "nsplit": out[1], "chunk": out[2], "block": out[3],
            "nstate": out[4]}


def decode_hpw(path: int) -> int:
    """KV heads per split workgroup of a decode plan path: 4/2/1 for the MFMA
    paths 1/2/3, 0 for the generic kernel."""
    return {1: 4, 2: 2, 3: 1}.get(int(path), 0)


def prefill_plan(q, k, v, out, num_heads, num_kv_heads, head_dim, q_stride=0, kv_stride=0):
    return int(lib().attn_prefill_plan(_ptr(q), _ptr(k), _ptr(v), _ptr(out), num_heads,
                                       num_kv_heads, head_dim, q_stride, kv_stride))


def decode_workspace(num_heads: int, kv_len: int, head_dim: int, device="cuda"):
    """Allocate the reference-sized decode workspace (model_inference.hpp:192-198)."""
    states = decode_workspace_states(num_heads, kv_len)
    return (torch.empty(states * head_dim, dtype=torch.float32, device=device),
            torch.empty(states, dtype=torch.float32, device=device),
            torch.empty(states, dtype=torch.float32, device=device))


class KVCache:
    """Device KV cache with the reference layout (kv_cache.hpp:8-83): one buffer for
    all layers; layer l holds K [S][Hkv*D] then V [S][Hkv*D]."""

    def __init__(self, num_layers, max_seq_len, num_kv_heads, head_dim, device="cuda",
                 fill=None):
        self.num_layers = num_layers
        self.max_seq_len = max_seq_len
        self.kv_dim = num_kv_heads * head_dim
        total = 2 * self.kv_dim * max_seq_len * num_layers
        if fill is None:
            self.buffer = torch.empty(total, dtype=torch.float16, device=device)
        else:
            self.buffer = torch.full((total,), fill, dtype=torch.float16, device=device)
        self.cached_len = 0

    def layer_stride(self):
        return 2 * self.kv_dim * self.max_seq_len

    def k(self, layer):
        o = layer * self.layer_stride()
        return self.buffer[o:o + self.max_seq_len * self.kv_dim].view(self.max_seq_len, self.kv_dim)

    def v(self, layer):
        o = layer * self.layer_stride() + self.max_seq_len * self.kv_dim
        return self.buffer[o:o + self.max_seq_len * self.kv_dim].view(self.max_seq_len, self.kv_dim)

    def set_cached_len(self, n):
        if n > self.max_seq_len:  # kv_cache.hpp:40-45
            raise IndexError(f"KV cache capacity exceeded: requested {n} tokens, capacity "
                             f"{self.max_seq_len}")
        self.cached_len = n


def _weights_error(rc: int, what: str):
    msg = lib().attn_weights_error_string(rc)
    raise AttnError(f"{what}: " + (msg.decode() if msg else f"hipError {rc}"))


def weights_parse(head: bytes, file_bytes: int) -> WeightsLayout:
    """Layout of a weights.bin of file_bytes bytes from its first bytes (at least
    48: the header and the tokenizer length); raises AttnError with the
    reference's message on a malformed file (model.hpp:40-93)."""
    lay = WeightsLayout()
    buf = ctypes.create_string_buffer(bytes(head), len(head))
    rc = lib().attn_weights_parse(ctypes.addressof(buf), len(head), file_bytes, ctypes.byref(lay))
    if rc != 0:
        _weights_error(rc, "attn_weights_parse")
    return lay


def weights_layout_for(config: ModelConfigC, payload_bytes: int) -> WeightsLayout:
    lay = WeightsLayout()
    rc = lib().attn_weights_layout_for(ctypes.byref(config), payload_bytes, ctypes.byref(lay))
    if rc != 0:
        _weights_error(rc, "attn_weights_layout_for")
    return lay


class ModelWeights:
    """A weights.bin in device memory the way the engine holds it
    (model.hpp:18-32, device_weights.hpp:57-110): the whole fp16 payload in one
    allocation, tensors addressed by offsets into it.  `qkv(l)` is layer l's
    fused [Hq*D + 2*Hkv*D][hidden] QKV weight (q_proj, k_proj, v_proj
    adjacent), the matrix the QKV projections take."""

    def __init__(self, path, device="cuda"):
        path = pathlib.Path(path)
        size = path.stat().st_size
        with open(path, "rb") as f:
            head = f.read(48)
        self.layout = weights_parse(head, size)
        lay = self.layout
        self.config = lay.config
        with open(path, "rb") as f:
            f.seek(lay.tokenizer_offset)
            self.tokenizer_json = f.read(lay.tokenizer_bytes)
        n = lay.weights_bytes // 2
        self.buffer = torch.empty(n, dtype=torch.float16, device=device)
        # streamed through one 64 MiB pinned buffer: the file is never held
        # whole in host memory; each copy completes before the buffer is reused
        chunk = min(n, 32 << 20)
        stage = torch.empty(chunk, dtype=torch.float16, pin_memory=True)
        raw = memoryview(stage.numpy()).cast("B")
        with open(path, "rb") as f:
            f.seek(lay.weights_offset)
            for o in range(0, n, chunk):
                c = min(chunk, n - o)
                got = 0
                while got < 2 * c:
                    r = f.readinto(raw[got:2 * c])
                    if not r:
                        raise AttnError(f"{path}: payload ended early")
                    got += r
                self.buffer[o:o + c].copy_(stage[:c])

    def _view(self, offset, *shape):
        n = math.prod(shape)
        return self.buffer[offset:offset + n].view(*shape)

    def layer(self, l, field):
        """Offset (elements) of a per-layer tensor (WEIGHT_LAYER_FIELDS)."""
        lay = self.layout
        if not 0 <= l < lay.config.num_layers:
            raise IndexError(l)
        rel = getattr(lay, field)
        if rel == 2**64 - 1:
            raise KeyError(f"{field} is not in this file")
        return lay.layer_base + l * lay.layer_elems + rel

    def qkv(self, l):
        c = self.config
        rows = (c.num_heads + 2 * c.num_kv_heads) * c.head_dim
        return self._view(self.layer(l, "q_proj"), rows, c.hidden_size)


def scale(head_dim: int) -> float:
    return 1.0 / math.sqrt(head_dim)
