"""weights.bin writer: a restatement of the reference exporter's byte format.

TEST INFRASTRUCTURE ONLY: imported by tests/ to make synthetic model files and
to state where each tensor lands; the product library never uses it.

Follows python/export_weights.py of MarcVivas/llm-inference:
* header: struct "<4sIIIIIIIIff" = b"QWEN", vocab_size, hidden_size,
  num_layers, num_heads, num_kv_heads, head_dim, intermediate_size,
  max_seq_len, rms_norm_eps, rope_theta (:51-68), 44 bytes;
* uint32 tokenizer-JSON length, the JSON bytes (:80-81);
* zero padding to a 64-byte file offset (:83-87);
* fp16 tensors, C order, in this order (:89-134): embedding; per layer
  input_layernorm, q_proj, k_proj, v_proj, [q_norm, k_norm if present],
  o_proj, post_attention_layernorm, gate_proj, up_proj, down_proj; final
  norm; lm_head (the embedding again when tied).
Shapes are Hugging Face's (nn.Linear weights are [out_features][in_features]).
The offsets are taken from the file position as each tensor is written, not
from a size formula, so a test comparing them with the library's layout checks
the layout against the write order itself.
"""
from __future__ import annotations

import struct

import numpy as np

HEADER = "<4sIIIIIIIIff"
SMOLLM3_3B = dict(vocab_size=128256, hidden_size=2048, num_layers=36, num_heads=16,
                  num_kv_heads=4, head_dim=128, intermediate_size=11008, max_seq_len=65536,
                  rms_norm_eps=1e-6, rope_theta=5.0e6)
CONFIG_FIELDS = ("vocab_size", "hidden_size", "num_layers", "num_heads", "num_kv_heads",
                 "head_dim", "intermediate_size", "max_seq_len", "rms_norm_eps", "rope_theta")


def tensor_shapes(cfg, qk_norm=False):
    """(name, shape) in the exporter's write order (export_weights.py:89-134)."""
    H, D, I, V = cfg["hidden_size"], cfg["head_dim"], cfg["intermediate_size"], cfg["vocab_size"]
    q_dim, kv_dim = cfg["num_heads"] * D, cfg["num_kv_heads"] * D
    out = [("model.embed_tokens.weight", (V, H))]
    for i in range(cfg["num_layers"]):
        p = f"model.layers.{i}."
        out += [(p + "input_layernorm.weight", (H,)),
                (p + "self_attn.q_proj.weight", (q_dim, H)),
                (p + "self_attn.k_proj.weight", (kv_dim, H)),
                (p + "self_attn.v_proj.weight", (kv_dim, H))]
        if qk_norm:
            out += [(p + "self_attn.q_norm.weight", (D,)), (p + "self_attn.k_norm.weight", (D,))]
        out += [(p + "self_attn.o_proj.weight", (H, q_dim)),
                (p + "post_attention_layernorm.weight", (H,)),
                (p + "mlp.gate_proj.weight", (I, H)),
                (p + "mlp.up_proj.weight", (I, H)),
                (p + "mlp.down_proj.weight", (H, I))]
    out += [("model.norm.weight", (H,)), ("lm_head.weight", (V, H))]
    return out


def header_bytes(cfg, magic=b"QWEN"):
    return struct.pack(HEADER, magic, *(cfg[f] for f in CONFIG_FIELDS))


def write(path, cfg, tokenizer_json: bytes, seed=0, qk_norm=False, tensors=None,
          trailing: bytes = b""):
    """Writes a weights.bin for cfg; tensors (name -> fp16 array) default to
    seeded N(0, 1/fan_in) values.  Returns (weights_offset, {name: (byte offset
    from the payload start, shape)})."""
    rng = np.random.default_rng(seed)
    where = {}
    with open(path, "wb") as f:
        f.write(header_bytes(cfg))
        f.write(struct.pack("<I", len(tokenizer_json)))
        f.write(tokenizer_json)
        f.write(b"\x00" * ((64 - f.tell() % 64) % 64))
        base = f.tell()
        for name, shape in tensor_shapes(cfg, qk_norm):
            if tensors is not None and name in tensors:
                t = np.asarray(tensors[name], dtype=np.float16)
                assert t.shape == shape, (name, t.shape, shape)
            else:
                scale = 1.0 / np.sqrt(shape[-1])
                t = (rng.standard_normal(shape, dtype=np.float32) * scale).astype(np.float16)
            where[name] = (f.tell() - base, shape)
            np.ascontiguousarray(t).tofile(f)
        f.write(trailing)
    return base, where


def payload_elements(cfg, qk_norm=False):
    return sum(int(np.prod(s)) for _, s in tensor_shapes(cfg, qk_norm))


def read_tensor(path, weights_offset, where, name):
    """The fp16 bit patterns (uint16) of one tensor, read back from the file."""
    off, shape = where[name]
    n = int(np.prod(shape))
    a = np.fromfile(path, dtype=np.uint16, count=n, offset=weights_offset + off)
    return a.reshape(shape)
