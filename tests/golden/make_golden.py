"""Writes the golden fixtures in tests/golden/ (run: python tests/golden/make_golden.py).

Every expected value here comes from an implementation that is independent of
the C oracle under test:
  * kat_flash_decode.npz -- the reference's Flash-Decode known-answer test
    (tests/test_causal_attention.cpp:152-228): inputs are the reference's
    closed forms (generated with libm sinf/cosf through the oracle's
    orc_kat_inputs, exactly as the reference test does on its host), expected
    outputs from a numpy float64 softmax written here.
  * rope.npz -- RoPE tables (numpy float64 cos/sin of the fp32 angle) and
    rotated Q/K from numpy float32 arithmetic (one rounding per product and
    per sum, as rope.hip.cpp:53-57 is written), for SmolLM3's theta = 5e6 at
    positions {0, 1, 2, 253, 32768}.
  * attention.npz -- seeded random causal GQA prefill and decode cases with
    expected outputs from torch (float64 matmul + softmax on the CPU, a library
    restatement of python/reference.py:79-92's SDPA + repeat_interleave).
The reference's own Python (python/reference.py) is read, never run: it needs a
network model download.
"""
from __future__ import annotations

import hashlib
import pathlib
import sys

import numpy as np
import torch

HERE = pathlib.Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT / "oracle"))
import oracle  # noqa: E402

KAT_LENGTHS = [1, 12, 13, 37, 257]  # test_causal_attention.cpp:154 (KV_CHUNK = 12)


def h2f(a):
    return np.asarray(a, dtype=np.uint16).view(np.float16).astype(np.float64)


def f64_to_f16_bits(x):
    # double -> float -> half, the order of test_causal_attention.cpp:194
    return np.asarray(x, dtype=np.float64).astype(np.float32).astype(np.float16).view(np.uint16)


def kat_cases():
    for head_dim in (32, 128):
        for kv_heads in (1, 2, 4):
            for length in KAT_LENGTHS:
                for padded in (False, True):
                    yield head_dim, kv_heads, length, padded


def kat_expected(q, k, v, heads, head_dim, kv_heads, length, stride):
    """numpy fp64 restatement of test_causal_attention.cpp:176-196."""
    qf, kf, vf = h2f(q), h2f(k), h2f(v)
    out = np.empty(heads * head_dim, dtype=np.float64)
    for h in range(heads):
        kh = h // (heads // kv_heads)
        qh = qf[h * head_dim:(h + 1) * head_dim]
        rows = np.arange(length)[:, None] * stride + kh * head_dim + np.arange(head_dim)[None, :]
        kk, vv = kf[rows], vf[rows]
        scores = (kk @ qh) / np.sqrt(head_dim)
        w = np.exp(scores - scores.max())
        out[h * head_dim:(h + 1) * head_dim] = (w @ vv) / w.sum()
    return f64_to_f16_bits(out)


def make_kat():
    data = {}
    heads = 4
    for head_dim, kv_heads, length, padded in kat_cases():
        kv_dim = kv_heads * head_dim
        stride = kv_dim + (17 if padded else 0)
        q, k, v = oracle.kat_inputs(heads, head_dim, kv_heads, length, stride)
        key = f"d{head_dim}_kv{kv_heads}_len{length}_pad{int(padded)}"
        data[key + "_expected"] = kat_expected(q, k, v, heads, head_dim, kv_heads, length, stride)
        digest = hashlib.sha256(q.tobytes() + k.tobytes() + v.tobytes()).hexdigest()[:16]
        data[key + "_inputs_sha"] = np.frombuffer(digest.encode(), dtype=np.uint8)
    np.savez_compressed(HERE / "kat_flash_decode.npz", **data)


def make_rope():
    theta, head_dim = 5.0e6, 128
    half = head_dim // 2
    positions = np.array([0, 1, 2, 253, 32768], dtype=np.int64)
    i = np.arange(half)
    exponent = (2 * i).astype(np.float32) / np.float32(head_dim)
    # correctly rounded fp32 pow (float64 pow of the fp32 operands, rounded once);
    # numpy's own float32 power is off by one ulp for some exponents
    pw = np.power(np.float64(np.float32(theta)), exponent.astype(np.float64)).astype(np.float32)
    inv_freq = np.float32(1.0) / pw
    angle = positions[:, None].astype(np.float32) * inv_freq[None, :]  # fp32 product
    cos16 = np.cos(angle.astype(np.float64)).astype(np.float32).astype(np.float16)
    sin16 = np.sin(angle.astype(np.float64)).astype(np.float32).astype(np.float16)
    rng = np.random.default_rng(7)
    heads = 20  # 16 Q heads + 4 K heads per token
    x = rng.standard_normal((len(positions), heads, head_dim)).astype(np.float16)
    x0 = x[:, :, :half].astype(np.float32)
    x1 = x[:, :, half:].astype(np.float32)
    c = cos16.astype(np.float32)[:, None, :]
    s = sin16.astype(np.float32)[:, None, :]
    o0 = (x0 * c - x1 * s).astype(np.float16)  # float32 ops, each rounded once
    o1 = (x1 * c + x0 * s).astype(np.float16)
    rot = np.concatenate([o0, o1], axis=2)
    np.savez_compressed(HERE / "rope.npz", theta=np.float64(theta), head_dim=np.int64(head_dim),
                        positions=positions, cos=cos16.view(np.uint16), sin=sin16.view(np.uint16),
                        x=x.view(np.uint16), rotated=rot.view(np.uint16))


def torch_attention(q, k, v, causal):
    """q [T, Hq, D], k/v [L, Hkv, D] float64 -> [T, Hq, D]; repeat_interleave GQA
    (python/reference.py:83-92), decode rows see every key."""
    T, Hq, D = q.shape
    Hkv = k.shape[1]
    kk = k.repeat_interleave(Hq // Hkv, dim=1)
    vv = v.repeat_interleave(Hq // Hkv, dim=1)
    s = torch.einsum("thd,lhd->htl", q, kk) / np.sqrt(D)
    if causal:
        L = k.shape[0]
        mask = torch.ones(T, L, dtype=torch.bool).triu(1)
        s = s.masked_fill(mask[None], float("-inf"))
    p = torch.softmax(s, dim=-1)
    return torch.einsum("htl,lhd->thd", p, vv)


def make_attention():
    data = {}
    rng = np.random.default_rng(11)
    # prefill cases: (N, Hq, Hkv, D)
    for name, (N, Hq, Hkv, D) in {"prefill_a": (33, 8, 2, 128), "prefill_b": (40, 4, 4, 32),
                                   "prefill_c": (9, 16, 4, 128)}.items():
        q = rng.standard_normal((N, Hq, D)).astype(np.float16)
        k = rng.standard_normal((N, Hkv, D)).astype(np.float16)
        v = rng.standard_normal((N, Hkv, D)).astype(np.float16)
        o = torch_attention(torch.from_numpy(q.astype(np.float64)),
                            torch.from_numpy(k.astype(np.float64)),
                            torch.from_numpy(v.astype(np.float64)), True).numpy()
        data[name + "_q"] = q.view(np.uint16)
        data[name + "_k"] = k.view(np.uint16)
        data[name + "_v"] = v.view(np.uint16)
        data[name + "_expected"] = f64_to_f16_bits(o)
    for name, (L, Hq, Hkv, D) in {"decode_a": (40, 16, 4, 128), "decode_b": (1, 16, 4, 128),
                                   "decode_c": (45, 8, 1, 64)}.items():
        q = rng.standard_normal((1, Hq, D)).astype(np.float16)
        k = rng.standard_normal((L, Hkv, D)).astype(np.float16)
        v = rng.standard_normal((L, Hkv, D)).astype(np.float16)
        o = torch_attention(torch.from_numpy(q.astype(np.float64)),
                            torch.from_numpy(k.astype(np.float64)),
                            torch.from_numpy(v.astype(np.float64)), False).numpy()
        data[name + "_q"] = q.view(np.uint16)
        data[name + "_k"] = k.view(np.uint16)
        data[name + "_v"] = v.view(np.uint16)
        data[name + "_expected"] = f64_to_f16_bits(o)
    np.savez_compressed(HERE / "attention.npz", **data)


if __name__ == "__main__":
    make_kat()
    make_rope()
    make_attention()
    for f in sorted(HERE.glob("*.npz")):
        print(f.name, f.stat().st_size)
