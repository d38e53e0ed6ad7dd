"""Pins the CPU oracle (oracle/attn_oracle.c) before it is trusted as the checker.

Each check is chosen so that a plausible mistake in the restatement (a wrong
rounding, a swapped rotation sign, a dropped merge rescale, an off-by-one in
the causal mask or the GQA head map) fails it.  CPU only.
"""
import numpy as np
import pytest

import oracle
from helpers import f16, ulp_diff

# ------------------------------------------------------------------ fp16 ---


def test_f16_to_f32_exhaustive_matches_numpy():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ours = oracle.f16_to_f32(bits)
    ref = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(ours), nan)
    assert np.array_equal(ours[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f32_to_f16_rounding_matches_numpy():
    rng = np.random.default_rng(0)
    # every fp16 value, the midpoints between neighbours (ties -> even), and
    # random floats across the whole range including subnormals and overflow
    h = np.arange(0x7c00, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float64)
    mids = (h[:-1] + h[1:]) / 2
    rand = np.concatenate([
        rng.standard_normal(200000) * 10.0 ** rng.integers(-9, 6, 200000),
        np.array([65504.0, 65519.99, 65520.0, 1e6, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26,
                  2.0 ** -14, 2.0 ** -14 - 2.0 ** -25, 0.0, -0.0, np.inf, -np.inf]),
    ])
    vals = np.concatenate([h, mids, -mids, rand]).astype(np.float32)
    ours = oracle.f32_to_f16(vals)
    ref = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(ours, ref)

# ------------------------------------------------------------------ RoPE ---


def test_rope_tables_match_golden(golden):
    g = golden("rope.npz")
    theta, D = float(g["theta"]), int(g["head_dim"])
    pos = g["positions"]
    c, s = oracle.rope_tables(int(pos.max()) + 1, D, theta)
    # fp32 libm vs fp64 numpy evaluation of the same fp32 angle: same fp16 up to
    # one ulp on rounding-boundary cases
    assert ulp_diff(c[pos], g["cos"]).max() <= 1
    assert ulp_diff(s[pos], g["sin"]).max() <= 1
    assert (ulp_diff(c[pos], g["cos"]) == 0).mean() > 0.98
    # position 0 is exactly (cos, sin) = (1, 0)
    assert np.all(c[0] == 0x3C00) and np.all(s[0] == 0)


def test_rope_inverse_frequencies_closed_form():
    # theta^(-2i/D): i = 0 -> 1 (angle = pos), so cos/sin of column 0 follow the
    # position directly; a wrong exponent (i/D, or 2i/(D-1)) breaks column 1
    D, theta = 128, 5.0e6
    c, s = oracle.rope_tables(4, D, theta)
    assert f16(c[1, 0]) == np.float16(np.cos(1.0)) and f16(s[1, 0]) == np.float16(np.sin(1.0))
    w1 = theta ** (-2.0 / D)
    assert abs(float(f16(s[3, 1])) - np.sin(3 * w1)) < 1e-3
    assert abs(float(f16(c[3, 1])) - np.cos(3 * w1)) < 1e-3


def _rope_setup(g):
    pos = g["positions"]
    c, s = oracle.rope_tables(int(pos.max()) + 1, 128, float(g["theta"]))
    return pos, c, s


def test_rope_rotation_bitexact_vs_numpy_golden(golden):
    g = golden("rope.npz")
    pos, c, s = _rope_setup(g)
    x = g["x"]  # [P, 20 heads, 128]
    for i, p in enumerate(pos):
        # rotate the 16 Q heads in place and the 4 K heads into a cache row
        q = np.ascontiguousarray(x[i, :16].reshape(-1))
        k = np.ascontiguousarray(x[i, 16:].reshape(-1))
        v = np.arange(512, dtype=np.uint16)
        kc = np.full(((p + 1) * 512,), 0xD7B0, dtype=np.uint16)
        vc = kc.copy()
        oracle.rope_store_kv(q, k, v, kc, vc, c, s, 1, 16, 4, 128, 2048, 512, int(p), True)
        assert np.array_equal(q.reshape(16, 128), g["rotated"][i, :16])
        assert np.array_equal(kc[p * 512:].reshape(4, 128), g["rotated"][i, 16:])
        assert np.array_equal(vc[p * 512:], v)
        assert np.array_equal(k, x[i, 16:].reshape(-1))  # K source unchanged


def _rotations(x, c, s):
    """out0 = x0 c - x1 s, out1 = x1 c + x0 s (rope.hip.cpp:44-58) in fp32 with
    every product rounded, and with either product of each output fused into
    an FMA (evaluated exactly in fp64, rounded once to fp32): all as fp16 bits."""
    x0, x1 = x[..., :64], x[..., 64:]
    p = {"x0c": x0 * c, "x1s": x1 * s, "x1c": x1 * c, "x0s": x0 * s}   # fp32-rounded
    e = {"x0c": x0.astype(np.float64) * c, "x1s": x1.astype(np.float64) * s,
         "x1c": x1.astype(np.float64) * c, "x0s": x0.astype(np.float64) * s}

    def bits(lo, hi):
        return np.concatenate([lo.astype(np.float32).astype(np.float16),
                               hi.astype(np.float32).astype(np.float16)], axis=-1).view(np.uint16)

    plain = bits(p["x0c"] - p["x1s"], p["x1c"] + p["x0s"])
    fused = [bits(e["x0c"] - p["x1s"], e["x1c"] + p["x0s"]),   # first product fused
             bits(-e["x1s"] + p["x0c"], e["x0s"] + p["x1c"])]  # second product fused
    return plain, fused


def test_rope_contracted_rotation_is_bit_identical(golden):
    """This build (kernels and oracle) computes rotate_pair with every product
    rounded; the reference is compiled by hipcc with clang's default FP
    contraction (xmake.lua:41, :80, :90 pass no -ffp-contract), which may fuse
    a product with the subtraction/addition into one FMA.  That cannot change
    the result: x, cos and sin are fp16 values (11 significant bits), so each
    fp32 product has at most 22 significant bits and is exact, and
    round(round(a c) + t) = round(a c + t).  Checked on rope.npz's inputs
    (positions 0, 1, 2, 253, 32768, theta 5e6, 20 heads) and on a million
    random fp16 values at random table rows up to 32768."""
    g = golden("rope.npz")
    x = f16(g["x"]).astype(np.float32)                    # [P, 20, 128]
    c = f16(g["cos"]).astype(np.float32)[:, None, :]      # [P, 1, 64]
    s = f16(g["sin"]).astype(np.float32)[:, None, :]
    plain, fused = _rotations(x, c, s)
    assert np.array_equal(plain, g["rotated"])            # the unfused form is the golden one
    for f in fused:
        assert np.array_equal(f, plain)
    cos, sin = oracle.rope_tables(32769, 128, 5.0e6)
    rng = np.random.default_rng(7)
    pos = rng.integers(0, 32769, 2048)
    c = f16(cos.reshape(32769, 64)[pos]).astype(np.float32)[:, None, :]
    s = f16(sin.reshape(32769, 64)[pos]).astype(np.float32)[:, None, :]
    x = (rng.standard_normal((2048, 4, 128)) * 3).astype(np.float16).astype(np.float32)
    plain, fused = _rotations(x, c, s)
    for f in fused:
        assert np.array_equal(f, plain)


def test_rope_position_zero_is_identity_and_quarter_turn_swaps():
    rng = np.random.default_rng(1)
    D, half = 128, 64
    q = rng.standard_normal(2 * D).astype(np.float16).view(np.uint16)
    q0 = q.copy()
    cos = np.full((2, half), 0x3C00, dtype=np.uint16)  # cos = 1
    sin = np.zeros((2, half), dtype=np.uint16)
    k = np.zeros(D, dtype=np.uint16)
    oracle.rope_store_kv(q, k, None, None, None, cos, sin, 1, 2, 1, D, 2 * D, D, 0, True)
    assert np.array_equal(q, q0)
    # a quarter turn (cos 0, sin 1): out0 = -x1, out1 = x0 exactly
    cos[:] = 0
    sin[:] = 0x3C00
    oracle.rope_store_kv(q, k, None, None, None, cos, sin, 1, 2, 1, D, 2 * D, D, 0, True)
    qq = q.reshape(2, D)
    q0 = q0.reshape(2, D)
    assert np.array_equal(qq[:, :half], (q0[:, half:] ^ 0x8000))
    assert np.array_equal(qq[:, half:], q0[:, :half])


def test_rope_nope_copy_and_untouched_rows():
    # rope.hip.cpp:9-42 NoPE path: bit-exact copies, Q untouched, rows outside
    # [start_pos, start_pos + seq) untouched (test_rope.cpp:165-175 semantics)
    rng = np.random.default_rng(2)
    N, Hq, Hkv, D, S, start = 5, 4, 2, 32, 9, 2
    qkv_stride = Hq * D + 2 * Hkv * D
    buf = rng.standard_normal(N * qkv_stride).astype(np.float16).view(np.uint16)
    orig = buf.copy()
    q = buf[:]
    kc = np.full(S * Hkv * D, 0xD7B0, dtype=np.uint16)
    vc = kc.copy()
    cos, sin = oracle.rope_tables(S, D, 1e4)
    k = np.ascontiguousarray(buf.reshape(N, -1)[:, Hq * D:Hq * D + Hkv * D]).reshape(-1)
    v = np.ascontiguousarray(buf.reshape(N, -1)[:, Hq * D + Hkv * D:]).reshape(-1)
    oracle.rope_store_kv(q, k, v, kc, vc, cos, sin, N, Hq, Hkv, D, qkv_stride, Hkv * D, start,
                         False)
    assert np.array_equal(buf, orig)
    kc2 = kc.reshape(S, -1)
    assert np.array_equal(kc2[start:start + N], k.reshape(N, -1))
    assert np.array_equal(vc.reshape(S, -1)[start:start + N], v.reshape(N, -1))
    assert np.all(kc2[:start] == 0xD7B0) and np.all(kc2[start + N:] == 0xD7B0)

# ------------------------------------------------------------ attention ---


def test_kat_inputs_match_closed_form():
    # the reference's KAT inputs (test_causal_attention.cpp:167-175), recomputed
    # in float64: the oracle's fp32 libm version agrees to within one fp16 ulp
    heads, D, Hkv, L, stride = 4, 32, 2, 13, 2 * 32 + 17
    q, k, v = oracle.kat_inputs(heads, D, Hkv, L, stride)
    i = np.arange(heads * D)
    assert ulp_diff(q, np.float16(2 * np.sin((i + 1) * 0.37)).view(np.uint16)).max() <= 1
    kk = k.reshape(L + 2, stride)
    t, j = np.meshgrid(np.arange(L), np.arange(Hkv * D), indexing="ij")
    assert ulp_diff(kk[:L, :Hkv * D],
                    np.float16(3 * np.cos((t * Hkv * D + j + 1) * 0.13)).view(np.uint16)).max() <= 1
    assert np.all(kk[:, Hkv * D:] == np.float16(123).view(np.uint16))
    assert np.all(kk[L:] == np.float16(123).view(np.uint16))


@pytest.mark.parametrize("head_dim", [32, 128])
@pytest.mark.parametrize("kv_heads", [1, 2, 4])
def test_oracle_decode_matches_reference_kat(golden, head_dim, kv_heads):
    g = golden("kat_flash_decode.npz")
    import hashlib
    heads = 4
    for length in (1, 12, 13, 37, 257):
        for padded in (0, 1):
            stride = kv_heads * head_dim + (17 if padded else 0)
            q, k, v = oracle.kat_inputs(heads, head_dim, kv_heads, length, stride)
            key = f"d{head_dim}_kv{kv_heads}_len{length}_pad{padded}"
            sha = hashlib.sha256(q.tobytes() + k.tobytes() + v.tobytes()).hexdigest()[:16]
            assert sha == bytes(g[key + "_inputs_sha"]).decode(), key
            out16, _ = oracle.attention(q, k, v, 1, heads, kv_heads, head_dim, heads * head_dim,
                                        stride, length, length - 1, causal=False)
            assert ulp_diff(out16.reshape(-1), g[key + "_expected"]).max() <= 1, key


@pytest.mark.parametrize("case", ["prefill_a", "prefill_b", "prefill_c"])
def test_oracle_prefill_matches_torch_golden(golden, case):
    g = golden("attention.npz")
    q, k, v, e = (g[f"{case}_{x}"] for x in ("q", "k", "v", "expected"))
    N, Hq, D = q.shape
    Hkv = k.shape[1]
    out16, _ = oracle.attention(q, k, v, N, Hq, Hkv, D, Hq * D, Hkv * D, N, causal=True)
    assert ulp_diff(out16, e).max() <= 1


@pytest.mark.parametrize("case", ["decode_a", "decode_b", "decode_c"])
def test_oracle_decode_matches_torch_golden(golden, case):
    g = golden("attention.npz")
    q, k, v, e = (g[f"{case}_{x}"] for x in ("q", "k", "v", "expected"))
    _, Hq, D = q.shape
    L, Hkv, _ = k.shape
    out16, _ = oracle.attention(q, k, v, 1, Hq, Hkv, D, Hq * D, Hkv * D, L, L - 1, causal=False)
    assert ulp_diff(out16, e).max() <= 1


def test_attention_closed_forms():
    rng = np.random.default_rng(3)
    Hq, Hkv, D, L = 4, 2, 16, 9
    q = rng.standard_normal(Hq * D).astype(np.float16).view(np.uint16)
    v = rng.standard_normal(L * Hkv * D).astype(np.float16).view(np.uint16)
    # one key: the output is V[0] exactly
    k = rng.standard_normal(L * Hkv * D).astype(np.float16).view(np.uint16)
    o, _ = oracle.attention(q, k, v, 1, Hq, Hkv, D, Hq * D, Hkv * D, 1, 0, causal=False)
    vv = v.reshape(L, Hkv, D)
    for h in range(Hq):
        assert np.array_equal(o[0, h], vv[0, h // 2])
    # identical keys: uniform weights, the output is the mean of V
    k1 = np.tile(k[:Hkv * D], L)
    _, o32 = oracle.attention(q, k1, v, 1, Hq, Hkv, D, Hq * D, Hkv * D, L, L - 1, causal=False)
    mean = f16(vv).astype(np.float64).mean(axis=0)
    for h in range(Hq):
        assert np.allclose(o32[0, h], mean[h // 2], atol=1e-6)


def test_attention_two_key_closed_form_and_head_map():
    # two keys, scores s0 = q.k0/sqrt(D), s1 = q.k1/sqrt(D): out = sigmoid(s0-s1) v0 + ...
    D = 4
    q = np.float16([1, 0, 0, 0, 0, 2, 0, 0]).view(np.uint16)  # two query heads
    k = np.float16([2, 0, 0, 0, 0, 4, 0, 0]).view(np.uint16)  # rows k0, k1 (1 kv head)
    v = np.float16([1, 0, 0, 0, 0, 1, 0, 0]).view(np.uint16)
    _, o = oracle.attention(q, k, v, 1, 2, 1, D, 2 * D, D, 2, 1, causal=False)
    s_h0 = np.array([2.0, 0.0]) / 2.0
    s_h1 = np.array([0.0, 8.0]) / 2.0
    for h, s in enumerate((s_h0, s_h1)):
        w = np.exp(s - s.max())
        w /= w.sum()
        assert np.allclose(o[0, h], [w[0], w[1], 0, 0], atol=1e-7)
    # GQA map h // (Hq/Hkv): with 4 q heads and 2 kv heads, heads 2,3 read kv head 1
    q4 = np.zeros(4 * D, dtype=np.float16).view(np.uint16)
    kk = np.zeros(2 * 2 * D, dtype=np.uint16)
    vv = np.float16([1, 1, 1, 1, 5, 5, 5, 5, 1, 1, 1, 1, 5, 5, 5, 5]).view(np.uint16)
    _, o4 = oracle.attention(q4, kk, vv, 1, 4, 2, D, 4 * D, 2 * D, 2, 1, causal=False)
    assert np.allclose(o4[0, :2], 1.0) and np.allclose(o4[0, 2:], 5.0)


def test_causal_row_independent_of_future_rows():
    rng = np.random.default_rng(4)
    N, Hq, Hkv, D = 12, 4, 2, 16
    q = rng.standard_normal(N * Hq * D).astype(np.float16).view(np.uint16)
    k = rng.standard_normal(N * Hkv * D).astype(np.float16).view(np.uint16)
    v = rng.standard_normal(N * Hkv * D).astype(np.float16).view(np.uint16)
    o, _ = oracle.attention(q, k, v, N, Hq, Hkv, D, Hq * D, Hkv * D, N, causal=True)
    t = 5
    k2, v2 = k.copy().reshape(N, -1), v.copy().reshape(N, -1)
    k2[t + 1:] = np.float16(123).view(np.uint16)
    v2[t + 1:] = np.float16(-77).view(np.uint16)
    o2, _ = oracle.attention(q, k2.reshape(-1), v2.reshape(-1), N, Hq, Hkv, D, Hq * D, Hkv * D,
                             N, causal=True)
    assert np.array_equal(o[:t + 1], o2[:t + 1])
    assert not np.array_equal(o[t + 1:], o2[t + 1:])
    # row 0 sees only key 0
    vv = v.reshape(N, Hkv, D)
    for h in range(Hq):
        assert np.array_equal(o[0, h], vv[0, h // 2])


@pytest.mark.parametrize("chunk", [1, 12, 13, 64, 300])
def test_chunked_merge_equals_full_softmax(chunk):
    # causal_attention.hip.cpp:719-838: per-chunk (max, sum, acc) merged with
    # exp(m_c - M) rescaling; the KAT inputs give chunks different maxima, so a
    # merge without the rescale is far off
    heads, D, Hkv, L = 4, 32, 2, 257
    stride = Hkv * D + 17
    q, k, v = oracle.kat_inputs(heads, D, Hkv, L, stride)
    _, full = oracle.attention(q, k, v, 1, heads, Hkv, D, heads * D, stride, L, L - 1,
                               causal=False)
    part = oracle.attention_chunked(q, k, v, heads, Hkv, D, stride, L, chunk)
    assert np.abs(part - full.reshape(heads, D)).max() < 2e-5


def test_kv_cache_offsets():
    # kv_cache.hpp:20-34, :71-82 for the SmolLM3 decode configuration
    S, Hkv, D = 32769, 4, 128
    ko, vo = oracle.kv_offsets(1, S, Hkv, D)
    assert ko == 2 * S * Hkv * D and vo == ko + S * Hkv * D
    assert oracle.kv_total_bytes(36, S, Hkv, D) == 2415992832

# ------------------------------------------------------------------ GEMV ---


@pytest.mark.parametrize("out_dim,in_dim", [(37, 2048), (129, 129), (9, 2053), (300, 64),
                                            (1, 1)])
def test_gemv_matches_numpy_float64(out_dim, in_dim):
    # numpy's float64 product is an independent library evaluation; the shapes
    # are non-square so a transposed W cannot even be formed the same way
    rng = np.random.default_rng(out_dim * 7 + in_dim)
    w = (rng.standard_normal((out_dim, in_dim)) / np.sqrt(in_dim)).astype(np.float16)
    x = rng.standard_normal(in_dim).astype(np.float16)
    ours = oracle.gemv(w.view(np.uint16), x.view(np.uint16))
    ref = (w.astype(np.float64) @ x.astype(np.float64)).astype(np.float32).astype(np.float16)
    d = ulp_diff(ours, ref.view(np.uint16))
    assert d.max() <= 1 and (d == 0).mean() > 0.999


def test_gemv_identity_rows_copy_x():
    # W = [I; 2I] selects x exactly (and doubles it exactly), an off-by-one in
    # the row or column index breaks it
    n = 257
    x = np.random.default_rng(3).standard_normal(n).astype(np.float16)
    w = np.concatenate([np.eye(n), 2 * np.eye(n)]).astype(np.float16)
    y = oracle.gemv(w.view(np.uint16), x.view(np.uint16))
    assert np.array_equal(y[:n], x.view(np.uint16))
    assert np.array_equal(f16(y[n:]), (2 * x.astype(np.float32)).astype(np.float16))


def gemv_reference_inputs(out_dim, in_dim):
    """test_matrix_vec_mul.cpp:21-24 closed-form weights and input."""
    i = np.arange(out_dim * in_dim)
    w = (((i % 29) - 14) / 64.0).astype(np.float16).reshape(out_dim, in_dim)
    x = (((np.arange(in_dim) % 17) - 8) / 16.0).astype(np.float16)
    return w, x


@pytest.mark.parametrize("out_dim,in_dim", [(7, 31), (37, 2048), (19, 11008), (9, 2053),
                                            (3, 0)])
def test_gemv_reference_known_answers(out_dim, in_dim):
    # the reference test's own inputs and tolerance (test_matrix_vec_mul.cpp:52-60)
    w, x = gemv_reference_inputs(out_dim, in_dim)
    y = f16(oracle.gemv(w.view(np.uint16), x.view(np.uint16))).astype(np.float64)
    exp = w.astype(np.float64) @ x.astype(np.float64)
    assert np.all(np.abs(y - exp) <= 1e-3 + 1e-3 * np.abs(exp))


def test_gemv_beta_zero_is_gemv_and_zero_weights_keep_residual():
    rng = np.random.default_rng(12)
    w = (rng.standard_normal((70, 300)) / 17).astype(np.float16).view(np.uint16)
    x = rng.standard_normal(300).astype(np.float16).view(np.uint16)
    y = rng.standard_normal(70).astype(np.float16).view(np.uint16)
    # beta = 0 ignores y (NaN included: it is never read)
    nan = np.full(70, np.float16(np.nan).view(np.uint16), np.uint16)
    assert np.array_equal(oracle.gemv_beta(w, x, nan, 0.0), oracle.gemv(w, x))
    # W = 0: the residual alone, y itself for beta = 1, fp16(beta y) otherwise
    zero = np.zeros_like(w)
    assert np.array_equal(oracle.gemv_beta(zero, x, y, 1.0), y)
    exp = (np.float32(0.75) * f16(y).astype(np.float32)).astype(np.float16)
    assert np.array_equal(oracle.gemv_beta(zero, x, y, 0.75), exp.view(np.uint16))
    # against numpy float64 + the residual, rounded once (one fp16 ulp at most)
    ref = ((w.view(np.float16).astype(np.float64) @ x.view(np.float16).astype(np.float64))
           + f16(y).astype(np.float64)).astype(np.float16)
    assert ulp_diff(oracle.gemv_beta(w, x, y, 1.0), ref.view(np.uint16)).max() <= 1


def test_gemv_beta_rounds_once():
    # W x = 1 + 2^-11 (exact in fp32, a tie in fp16 that rounds to 1) and
    # y = 2^-12: the sum 1 + 3 * 2^-12 rounds once to 1 + 2^-10; rounding the
    # product to fp16 first would give 1 + 2^-12 -> 1
    w = np.array([[1.0, 2.0 ** -11]], np.float16).view(np.uint16)
    x = np.array([1.0, 1.0], np.float16).view(np.uint16)
    y = np.array([2.0 ** -12], np.float16).view(np.uint16)
    assert f16(oracle.gemv_beta(w, x, y, 1.0))[0] == np.float16(1 + 2.0 ** -10)
    assert f16(oracle.gemv(w, x))[0] == np.float16(1.0)
    # a small hand-worked case: [1 2] . [3 4] + 0.5 = 11.5
    w = np.array([[1.0, 2.0]], np.float16).view(np.uint16)
    x = np.array([3.0, 4.0], np.float16).view(np.uint16)
    y = np.array([0.5], np.float16).view(np.uint16)
    assert f16(oracle.gemv_beta(w, x, y, 1.0))[0] == np.float16(11.5)
    assert f16(oracle.gemv_beta(w, x, y, -2.0))[0] == np.float16(10.0)


def test_gemm_rows_match_gemv_and_numpy():
    # orc_gemm is orc_gemv per token row; against numpy float64 on a
    # non-square product (a transposed operand has the wrong shape)
    rng = np.random.default_rng(9)
    x = rng.standard_normal((37, 96)).astype(np.float16)
    w = (rng.standard_normal((50, 96)) / 10).astype(np.float16)
    y = oracle.gemm(x.view(np.uint16), w.view(np.uint16))
    assert y.shape == (37, 50)
    for m in (0, 17, 36):
        assert np.array_equal(y[m], oracle.gemv(w.view(np.uint16), x[m].view(np.uint16)))
    ref = (x.astype(np.float64) @ w.astype(np.float64).T).astype(np.float32).astype(np.float16)
    d = ulp_diff(y, ref.view(np.uint16))
    assert d.max() <= 1 and (d == 0).mean() > 0.999
