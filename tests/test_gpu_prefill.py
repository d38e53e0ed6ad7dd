"""Causal GQA prefill on the GPU vs the oracle (and, at 8192 tokens, vs a torch
fp32 reference computed on the GPU).

Engine layout as in model_inference.hpp:272-293: Q read in place from the fused
[N, 3072] QKV buffer (q_stride 3072), K/V from the KV cache (kv_stride 512)
whose rows past N hold sentinel 123.0 (test_causal_attention.cpp:31-50); the
test_qkv_gemm.cpp:86-116 chain reads K/V straight from the fused buffer.
Tolerance: |a - e| <= 2e-3 + 1e-2 |e| against the fp64 oracle."""
import numpy as np
import pytest
import torch

import oracle
from helpers import assert_close

pytestmark = pytest.mark.gpu


def dev(a, device):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.float16)).to(device)


def host(t):
    return t.detach().cpu().numpy().view(np.uint16)


def engine_inputs(N, seed, sigma=1.0, Hq=16, Hkv=4, D=128):
    rng = np.random.default_rng(seed)
    stride = Hq * D + 2 * Hkv * D
    qkv = (rng.standard_normal(N * stride) * sigma).astype(np.float16).view(np.uint16)
    cache = np.full(2 * (N + 2) * Hkv * D, np.float16(123.0).view(np.uint16), dtype=np.uint16)
    rows = qkv.reshape(N, stride)
    kc = cache[:(N + 2) * Hkv * D].reshape(N + 2, Hkv * D)
    vc = cache[(N + 2) * Hkv * D:].reshape(N + 2, Hkv * D)
    kc[:N] = rows[:, Hq * D:Hq * D + Hkv * D]
    vc[:N] = rows[:, Hq * D + Hkv * D:]
    return qkv, cache, stride


def run_prefill(attn, device, qkv, cache, N, stride, Hq=16, Hkv=4, D=128, from_cache=True):
    kv_dim = Hkv * D
    d_qkv, d_cache = dev(qkv, device), dev(cache, device)
    out = torch.empty(N * Hq * D, dtype=torch.float16, device=device)
    b, cb = d_qkv.data_ptr(), d_cache.data_ptr()
    if from_cache:
        attn.prefill(b, cb, cb + 2 * (N + 2) * kv_dim, out, N, Hq, Hkv, D, stride, kv_dim)
    else:
        attn.prefill(b, b + 2 * Hq * D, b + 2 * (Hq * D + kv_dim), out, N, Hq, Hkv, D, stride,
                     stride)
    torch.cuda.synchronize()
    assert np.array_equal(host(d_qkv), qkv) and np.array_equal(host(d_cache), cache)
    return host(out)


def oracle_prefill(qkv, cache, N, stride, Hq=16, Hkv=4, D=128, rows=None):
    kv_dim = Hkv * D
    k = cache[:(N + 2) * kv_dim]
    v = cache[(N + 2) * kv_dim:]
    _, e32 = oracle.attention(qkv, k, v, N, Hq, Hkv, D, stride, kv_dim, N, causal=True,
                              rows=rows)
    return e32


@pytest.mark.parametrize("N", [1, 2, 31, 63, 64, 65, 128, 200, 254])
def test_prefill_engine_layout(attn, gpu, N):
    qkv, cache, stride = engine_inputs(N, seed=N)
    print(f"[case] prefill N={N} path={attn.prefill_plan(4096, 4096, 4096, 4096, 16, 4, 128, stride, 512)}",
          flush=True)
    got = run_prefill(attn, gpu, qkv, cache, N, stride)
    assert_close(got, oracle_prefill(qkv, cache, N, stride).reshape(-1), 2e-3, 1e-2, f"N={N}")


@pytest.mark.parametrize("N", [254, 2000])
def test_prefill_fused_buffer_chain(attn, gpu, N):
    # test_qkv_gemm.cpp:86-116: K/V read from the interleaved GEMM output
    # (2000 tokens: the key-halves tile, sampled rows)
    qkv, cache, stride = engine_inputs(N, seed=77 + N)
    got = run_prefill(attn, gpu, qkv, cache, N, stride, from_cache=False)
    rows = None if N <= 1024 else np.unique(np.concatenate([np.arange(0, N, 19), [N - 1]]))
    _, e32 = oracle.attention(qkv, qkv[2048:], qkv[2560:], N, 16, 4, 128, stride, stride, N,
                              causal=True, rows=rows)
    if rows is not None:
        got = got.reshape(N, -1)[rows].reshape(-1)
    assert_close(got, e32.reshape(-1), 2e-3, 1e-2, "chain")


def test_prefill_golden_fixtures(attn, gpu, golden):
    g = golden("attention.npz")
    for case in ("prefill_a", "prefill_b", "prefill_c"):
        q, k, v, e = (g[f"{case}_{x}"] for x in ("q", "k", "v", "expected"))
        N, Hq, D = q.shape
        Hkv = k.shape[1]
        print(f"[case] prefill golden {case} N={N} Hq={Hq} Hkv={Hkv} D={D}", flush=True)
        out = torch.empty(N * Hq * D, dtype=torch.float16, device=gpu)
        attn.prefill(dev(q, gpu), dev(k, gpu), dev(v, gpu), out, N, Hq, Hkv, D)
        torch.cuda.synchronize()
        assert_close(host(out), e.reshape(-1), 2e-3, 2e-3, case)


def test_prefill_8192_vs_oracle_rows_and_torch(attn, gpu):
    """C4: 8192 tokens, N(0, 0.5).  Sampled rows against the fp64 oracle, every
    row against a torch fp32 reference on the GPU (math path, row blocks)."""
    N, Hq, Hkv, D = 8192, 16, 4, 128
    qkv, cache, stride = engine_inputs(N, seed=4, sigma=0.5)
    print("[case] prefill N=8192", flush=True)
    got = run_prefill(attn, gpu, qkv, cache, N, stride)
    rows = np.unique(np.concatenate([np.arange(0, 70), np.arange(N - 70, N),
                                     np.arange(63, N, 512), np.arange(64, N, 1021)]))
    e_rows = oracle_prefill(qkv, cache, N, stride, rows=rows)
    got3 = got.reshape(N, Hq, D)
    assert_close(got3[rows].reshape(-1), e_rows.reshape(-1), 2e-3, 1e-2, "oracle rows")
    # torch fp32 reference for all rows
    x = torch.from_numpy(qkv.view(np.float16)).to(gpu).view(N, stride).float()
    q = x[:, :Hq * D].view(N, Hq, D).transpose(0, 1).contiguous()
    k = x[:, Hq * D:Hq * D + Hkv * D].view(N, Hkv, D).transpose(0, 1)
    v = x[:, Hq * D + Hkv * D:].view(N, Hkv, D).transpose(0, 1)
    k = k.repeat_interleave(Hq // Hkv, dim=0).contiguous()
    v = v.repeat_interleave(Hq // Hkv, dim=0).contiguous()
    ref = torch.empty(Hq, N, D, device=gpu)
    for r0 in range(0, N, 1024):
        r1 = r0 + 1024
        s = torch.matmul(q[:, r0:r1], k[:, :r1].transpose(1, 2).contiguous()) / np.sqrt(D)
        mask = torch.arange(r1, device=gpu)[None, :] > torch.arange(r0, r1, device=gpu)[:, None]
        s.masked_fill_(mask[None], float("-inf"))
        ref[:, r0:r1] = torch.matmul(torch.softmax(s, dim=-1), v[:, :r1])
    ref = ref.transpose(0, 1).contiguous().cpu().numpy().reshape(-1)
    assert_close(got, ref, 2e-3, 1e-2, "torch fp32")


@pytest.mark.parametrize("N,prefixes,split_keys", [(700, (1, 64, 65, 333), 1),
                                                   (254, (1, 31, 64, 65, 200), 2),
                                                   (254, (1, 31, 64, 65, 200), 3),
                                                   (700, (1, 31, 33, 64, 65, 333), 4)])
def test_prefill_prefix_invariance(attn, gpu, N, prefixes, split_keys):
    """Row t depends only on rows <= t: a prefill of N tokens and of a prefix
    of N' tokens agree bit for bit on the first N' rows -- across the
    pipelined and all-tiles-staged kernels (which compute the same tiles in
    the same order; the split-keys form is off), and within each split-keys
    form of short prompts (option value 2: 64-key tiles over 4 waves, 3:
    32-key units over 8 waves, 4: 32-key units streamed per wave; the same
    units combined the same way)."""
    qkv, cache, stride = engine_inputs(N, seed=21)
    try:
        attn.set_option("prefill_split_keys", split_keys)
        full = run_prefill(attn, gpu, qkv, cache, N, stride).reshape(N, -1)
        for Np in prefixes:
            print(f"[case] prefill prefix N={N} N'={Np} split_keys={split_keys}", flush=True)
            q2, c2, _ = engine_inputs(N, seed=21)
            c2 = np.concatenate([c2[:(N + 2) * 512].reshape(N + 2, 512)[:Np + 2].reshape(-1),
                                 c2[(N + 2) * 512:].reshape(N + 2, 512)[:Np + 2].reshape(-1)])
            part = run_prefill(attn, gpu, q2[:Np * stride], c2, Np, stride).reshape(Np, -1)
            assert np.array_equal(part, full[:Np]), Np
    finally:
        attn.set_option("prefill_split_keys", 0)


@pytest.mark.parametrize("Hq,Hkv,D,extra", [(16, 4, 64, 0), (16, 16, 128, 0), (8, 2, 128, 8),
                                            (16, 4, 128, 3), (6, 2, 32, 0)])
def test_prefill_generic_shapes(attn, gpu, Hq, Hkv, D, extra):
    N = 97
    rng = np.random.default_rng(D + Hq + extra)
    stride = Hq * D + 2 * Hkv * D + extra
    qkv = rng.standard_normal(N * stride).astype(np.float16).view(np.uint16)
    path = attn.prefill_plan(4096, 4096, 4096, 4096, Hq, Hkv, D, stride, stride)
    print(f"[case] prefill Hq={Hq} Hkv={Hkv} D={D} extra={extra} path={path}", flush=True)
    d = dev(qkv, gpu)
    out = torch.empty(N * Hq * D, dtype=torch.float16, device=gpu)
    b = d.data_ptr()
    attn.prefill(b, b + 2 * Hq * D, b + 2 * (Hq * D + Hkv * D), out, N, Hq, Hkv, D, stride,
                 stride)
    torch.cuda.synchronize()
    _, e32 = oracle.attention(qkv, qkv[Hq * D:], qkv[Hq * D + Hkv * D:], N, Hq, Hkv, D, stride,
                              stride, N, causal=True)
    assert_close(host(out), e32.reshape(-1), 2e-3, 1e-2, f"{Hq}/{Hkv}/{D}")


def test_prefill_forced_generic_matches_oracle(attn, gpu):
    N = 150
    qkv, cache, stride = engine_inputs(N, seed=5)
    attn.set_option("prefill_force_generic", 1)
    try:
        got = run_prefill(attn, gpu, qkv, cache, N, stride)
    finally:
        attn.set_option("prefill_force_generic", 0)
    assert_close(got, oracle_prefill(qkv, cache, N, stride).reshape(-1), 2e-3, 1e-2, "generic")


def test_prefill_beyond_c4_odd_length(attn, gpu):
    """N = 12289 (past C4, not a multiple of the 64-token tile): sampled rows,
    including the last partial tile, against the fp64 oracle."""
    N = 12289
    qkv, cache, stride = engine_inputs(N, seed=31, sigma=0.5)
    print(f"[case] prefill N={N}", flush=True)
    got = run_prefill(attn, gpu, qkv, cache, N, stride).reshape(N, -1)
    rows = np.array([0, 1, 63, 64, 4095, 8191, 8192, 12223, 12224, 12287, 12288])
    e_rows = oracle_prefill(qkv, cache, N, stride, rows=rows)
    assert_close(got[rows].reshape(-1), e_rows.reshape(-1), 2e-3, 1e-2, f"N={N}")


@pytest.mark.parametrize("Hq,Hkv", [(32, 4), (16, 2)])
def test_prefill_mfma_group_of_8(attn, gpu, Hq, Hkv):
    """GQA groups of 8 query heads per KV head take the MFMA path too."""
    N, D = 300, 128
    qkv, cache, stride = engine_inputs(N, seed=Hq + Hkv, Hq=Hq, Hkv=Hkv)
    assert attn.prefill_plan(4096, 4096, 4096, 4096, Hq, Hkv, D, stride, Hkv * D) == 1
    print(f"[case] prefill Hq={Hq} Hkv={Hkv} N={N}", flush=True)
    got = run_prefill(attn, gpu, qkv, cache, N, stride, Hq=Hq, Hkv=Hkv)
    e = oracle_prefill(qkv, cache, N, stride, Hq=Hq, Hkv=Hkv)
    assert_close(got, e.reshape(-1), 2e-3, 1e-2, f"{Hq}/{Hkv}")


@pytest.mark.parametrize("N", [333, 1500])
def test_prefill_mfma_padded_strides(attn, gpu, N):
    """Padded (8-element aligned) Q and K/V row strides stay on the MFMA path
    (333 tokens: the streaming split-keys form; 1500: the key-halves tile)."""
    Hq, Hkv, D = 16, 4, 128
    q_stride, kv_stride = Hq * D + 24, Hkv * D + 8
    rng = np.random.default_rng(41)
    q = rng.standard_normal(N * q_stride).astype(np.float16).view(np.uint16)
    k = rng.standard_normal((N + 1) * kv_stride).astype(np.float16).view(np.uint16)
    v = rng.standard_normal((N + 1) * kv_stride).astype(np.float16).view(np.uint16)
    assert attn.prefill_plan(4096, 4096, 4096, 4096, Hq, Hkv, D, q_stride, kv_stride) == 1
    print(f"[case] prefill padded strides q={q_stride} kv={kv_stride}", flush=True)
    out = torch.empty(N * Hq * D, dtype=torch.float16, device=gpu)
    attn.prefill(dev(q, gpu), dev(k, gpu), dev(v, gpu), out, N, Hq, Hkv, D, q_stride, kv_stride)
    torch.cuda.synchronize()
    rows = None if N <= 1024 else np.unique(np.concatenate([np.arange(0, N, 23), [N - 1]]))
    _, e32 = oracle.attention(q, k, v, N, Hq, Hkv, D, q_stride, kv_stride, N, causal=True,
                              rows=rows)
    got = host(out) if rows is None else host(out).reshape(N, -1)[rows].reshape(-1)
    assert_close(got, e32.reshape(-1), 2e-3, 1e-2, "padded strides")


@pytest.mark.parametrize("N", [1, 31, 32, 33, 64, 65, 96, 97, 254, 1000, 1023, 1024, 2049])
def test_prefill_four_and_eight_wave_tiles_identical(attn, gpu, N):
    """Short prompts run 32-query workgroups of 4 waves, long ones 64-query
    workgroups of 8 waves.  Each wave computes the same 32 queries over the
    same key tiles in the same order either way, so the two give the same
    bits (also past the diagonal of an odd 32-query tile and with the last
    query tile partly past N); and both equal the oracle within tolerance."""
    qkv, cache, stride = engine_inputs(N, seed=700 + N)
    outs = {}
    try:
        # the split-keys form of short prompts combines tiles in another order
        attn.set_option("prefill_split_keys", 1)
        for waves in (4, 8):
            attn.set_option("prefill_waves", waves)
            print(f"[case] prefill N={N} waves={waves}", flush=True)
            outs[waves] = run_prefill(attn, gpu, qkv, cache, N, stride)
    finally:
        attn.set_option("prefill_waves", 0)
        attn.set_option("prefill_split_keys", 0)
    assert np.array_equal(outs[4], outs[8])
    rows = None if N <= 1024 else np.unique(np.concatenate([np.arange(0, N, 7), [N - 1]]))
    exp = oracle_prefill(qkv, cache, N, stride, rows=rows).reshape(-1)
    got = outs[4] if rows is None else outs[4].reshape(N, -1)[rows].reshape(-1)
    assert_close(got, exp, 2e-3, 1e-2, f"N={N}")


@pytest.mark.parametrize("form", [0, 2, 3, 4])
@pytest.mark.parametrize("N", [1, 2, 31, 32, 33, 63, 64, 65, 96, 97, 128, 129, 191, 192, 200,
                               254, 255, 256])
def test_prefill_split_keys_vs_oracle(attn, gpu, N, form):
    """Short prompts (N <= 256): one workgroup per head and 32-query tile,
    its keys split over the waves (form 2: 64-key tiles over 4 waves; form
    3: 32-key units over 8 waves; form 4: 32-key units streamed per wave;
    form 0, the default: form 3 up to 32 tokens, form 2 above) and combined
    through LDS;
    against the fp64 oracle, and against the sequential kernel (the same
    attention, combined in another order: within the tolerance)."""
    qkv, cache, stride = engine_inputs(N, seed=1300 + N)
    print(f"[case] prefill split keys N={N} form={form}", flush=True)
    try:
        attn.set_option("prefill_split_keys", form)
        got = run_prefill(attn, gpu, qkv, cache, N, stride)
        attn.set_option("prefill_split_keys", 1)
        seq = run_prefill(attn, gpu, qkv, cache, N, stride)
    finally:
        attn.set_option("prefill_split_keys", 0)
    assert_close(got, oracle_prefill(qkv, cache, N, stride).reshape(-1), 2e-3, 1e-2, f"N={N}")
    assert_close(got, seq, 2e-3, 1e-2, f"N={N} vs sequential tiles")


@pytest.mark.parametrize("Hq,Hkv,N", [(8, 2, 256), (4, 1, 100), (32, 4, 97), (16, 2, 255)])
def test_prefill_split_keys_other_heads(attn, gpu, Hq, Hkv, N):
    """The split-keys forms at other head counts (4 and 8 query heads take
    the XCD-pinned block order, 16 and 32 the plain one) and with padded row
    strides, against the fp64 oracle."""
    D = 128
    q_stride, kv_stride = Hq * D + 8, Hkv * D + 24
    rng = np.random.default_rng(Hq * 1000 + N)
    q = rng.standard_normal(N * q_stride).astype(np.float16).view(np.uint16)
    k = rng.standard_normal((N + 1) * kv_stride).astype(np.float16).view(np.uint16)
    v = rng.standard_normal((N + 1) * kv_stride).astype(np.float16).view(np.uint16)
    _, e32 = oracle.attention(q, k, v, N, Hq, Hkv, D, q_stride, kv_stride, N, causal=True)
    try:
        for form in (2, 3, 4):
            attn.set_option("prefill_split_keys", form)
            print(f"[case] prefill split keys Hq={Hq} Hkv={Hkv} N={N} form={form}", flush=True)
            out = torch.empty(N * Hq * D, dtype=torch.float16, device=gpu)
            attn.prefill(dev(q, gpu), dev(k, gpu), dev(v, gpu), out, N, Hq, Hkv, D, q_stride,
                         kv_stride)
            torch.cuda.synchronize()
            assert_close(host(out), e32.reshape(-1), 2e-3, 1e-2, f"{Hq}/{Hkv} N={N} form={form}")
    finally:
        attn.set_option("prefill_split_keys", 0)


@pytest.mark.parametrize("N", [257, 288, 300, 511, 512, 640, 777, 1024, 1500, 1536, 1537, 2049])
def test_prefill_streaming_split_keys(attn, gpu, N):
    """Prompts past the all-tiles forms: one workgroup per head and 32-query
    tile whose 4 waves each stream every 4th 32-key unit (the default from
    257 to 1024 tokens, option value 4 at any length); against the fp64
    oracle (every row up to 1024 tokens, sampled rows above) and against the
    4-head kernels (the same attention, combined in another order)."""
    qkv, cache, stride = engine_inputs(N, seed=1700 + N)
    rows = None if N <= 1024 else np.unique(np.concatenate([np.arange(0, N, 13), [N - 1]]))
    exp = oracle_prefill(qkv, cache, N, stride, rows=rows).reshape(-1)
    outs = {}
    try:
        for form in (0, 4, 1):
            attn.set_option("prefill_split_keys", form)
            print(f"[case] prefill streaming split keys N={N} form={form}", flush=True)
            outs[form] = run_prefill(attn, gpu, qkv, cache, N, stride)
    finally:
        attn.set_option("prefill_split_keys", 0)
    if N <= 1024:
        assert np.array_equal(outs[0], outs[4])  # the default is the streaming form
    for form in (0, 4):
        got = outs[form] if rows is None else outs[form].reshape(N, -1)[rows].reshape(-1)
        assert_close(got, exp, 2e-3, 1e-2, f"N={N} form={form}")
    assert_close(outs[4], outs[1], 2e-3, 1e-2, f"N={N} vs the 4-head kernels")


def growing_score_inputs(N, seed, Hq=16, Hkv=4, D=128, beta=20.0):
    """Engine-layout inputs whose scores grow along the keys: every query row
    is g + noise and key row j is (j / N) beta g + noise for a fixed g of
    0.5s, so q.k rises by ~beta |g|^2 / N per key and a query's running
    maximum keeps moving past the lazy-rescale slack."""
    qkv, cache, stride = engine_inputs(N, seed)
    rng = np.random.default_rng(seed + 1)
    g = np.full(D, 0.5)
    rows = qkv.view(np.float16).reshape(N, stride)
    q = g + 0.3 * rng.standard_normal((N, Hq, D))
    k = (np.arange(N)[:, None, None] / N) * beta * g + 0.3 * rng.standard_normal((N, Hkv, D))
    rows[:, :Hq * D] = q.reshape(N, -1).astype(np.float16)
    rows[:, Hq * D:Hq * D + Hkv * D] = k.reshape(N, -1).astype(np.float16)
    kc = cache.view(np.float16)[:(N + 2) * Hkv * D].reshape(N + 2, Hkv * D)
    kc[:N] = rows[:, Hq * D:Hq * D + Hkv * D]
    return qkv, cache, stride


@pytest.mark.parametrize("N,waves,split_keys", [(254, 0, 0), (254, 4, 1), (254, 8, 1),
                                                (1000, 0, 0), (1000, 4, 1), (1000, 8, 1),
                                                (4096, 0, 0)])
def test_prefill_growing_scores_rescale(attn, gpu, N, waves, split_keys):
    """The running maximum moves past the slack on many key tiles (checked
    here on the inputs), so the rescale block -- which also shifts the tile's
    scores and the accumulators' starting value in the long-prompt tiles --
    runs again and again after the first tile; every form against the fp64
    oracle (sampled rows at 4096 tokens)."""
    qkv, cache, stride = growing_score_inputs(N, seed=900 + N)
    # the last query's maximum per 64-key tile, in exp2 units: count the
    # tiles whose maximum exceeds every earlier one by more than 8
    x = qkv.view(np.float16).reshape(N, stride).astype(np.float64)
    s = (x[N - 1, :128] @ x[:, 2048:2048 + 128].T) / np.sqrt(128) * np.log2(np.e)
    tmax = [s[j:j + 64].max() for j in range(0, N, 64)]
    m, moves = tmax[0], 0
    for t in tmax[1:]:
        if t > m + 8:
            m, moves = t, moves + 1
    assert moves >= (2 if N < 512 else 4), moves
    rows = None if N <= 1024 else np.unique(np.concatenate([np.arange(0, N, 37), [N - 1]]))
    exp = oracle_prefill(qkv, cache, N, stride, rows=rows).reshape(-1)
    try:
        attn.set_option("prefill_waves", waves)
        attn.set_option("prefill_split_keys", split_keys)
        print(f"[case] prefill growing scores N={N} waves={waves} split_keys={split_keys}",
              flush=True)
        got = run_prefill(attn, gpu, qkv, cache, N, stride)
    finally:
        attn.set_option("prefill_waves", 0)
        attn.set_option("prefill_split_keys", 0)
    if rows is not None:
        got = got.reshape(N, -1)[rows].reshape(-1)
    assert_close(got, exp, 2e-3, 1e-2, f"N={N} waves={waves} split_keys={split_keys}")


@pytest.mark.parametrize("N", [1, 31, 32, 33, 64, 65, 96, 254, 257, 700, 1025, 2049, 3000])
def test_prefill_key_halves(attn, gpu, N):
    """32-query tiles whose key tiles the two 4-wave groups of an 8-wave
    workgroup split (even and odd tiles, states combined through LDS; the
    default from 1025 to 4096 tokens, option value 2 at any length): against
    the fp64 oracle (sampled rows above 1024 tokens), against the 4-wave
    tiles, and with a query's row independent of what follows it."""
    qkv, cache, stride = engine_inputs(N, seed=2300 + N)
    rows = None if N <= 1024 else np.unique(np.concatenate([np.arange(0, N, 11), [N - 1]]))
    exp = oracle_prefill(qkv, cache, N, stride, rows=rows).reshape(-1)
    try:
        attn.set_option("prefill_key_halves", 2)
        print(f"[case] prefill key halves N={N}", flush=True)
        got = run_prefill(attn, gpu, qkv, cache, N, stride)
        if N > 64:
            # the first 64 tokens alone give the same rows
            q2, c2, _ = engine_inputs(64, seed=2300 + N)
            x = qkv.view(np.float16).reshape(N, stride)[:64].copy()
            q2 = x.reshape(-1).view(np.uint16)
            c2[:] = np.float16(123.0).view(np.uint16)
            kv = c2.view(np.float16)
            kv[:66 * 512].reshape(66, 512)[:64] = x[:, 2048:2560]
            kv[66 * 512:].reshape(66, 512)[:64] = x[:, 2560:]
            head = run_prefill(attn, gpu, q2, c2, 64, stride)
            assert np.array_equal(head, got.reshape(N, -1)[:64].reshape(-1))
        if 1024 < N <= 4096:
            attn.set_option("prefill_key_halves", 0)
            assert np.array_equal(run_prefill(attn, gpu, qkv, cache, N, stride), got)
        attn.set_option("prefill_key_halves", 1)
        attn.set_option("prefill_split_keys", 1)
        attn.set_option("prefill_waves", 4)
        ref = run_prefill(attn, gpu, qkv, cache, N, stride)
    finally:
        attn.set_option("prefill_key_halves", 0)
        attn.set_option("prefill_split_keys", 0)
        attn.set_option("prefill_waves", 0)
    g = got if rows is None else got.reshape(N, -1)[rows].reshape(-1)
    assert_close(g, exp, 2e-3, 1e-2, f"N={N}")
    assert_close(got, ref, 2e-3, 1e-2, f"N={N} vs the 4-wave tiles")


@pytest.mark.parametrize("Hq,Hkv,N", [(32, 4, 1500), (8, 2, 1100), (4, 1, 2049), (12, 3, 1300)])
def test_prefill_key_halves_other_heads(attn, gpu, Hq, Hkv, N):
    """The key-halves tile at other head counts (2, 8 and 3 head quads: the
    XCD-pinned and the plain workgroup orders), forced and as the default,
    against the fp64 oracle on sampled rows."""
    qkv, cache, stride = engine_inputs(N, seed=2500 + N, Hq=Hq, Hkv=Hkv)
    rows = np.unique(np.concatenate([np.arange(0, N, 17), [N - 1]]))
    exp = oracle_prefill(qkv, cache, N, stride, Hq=Hq, Hkv=Hkv, rows=rows).reshape(-1)
    try:
        attn.set_option("prefill_key_halves", 2)
        print(f"[case] prefill key halves Hq={Hq} Hkv={Hkv} N={N}", flush=True)
        got = run_prefill(attn, gpu, qkv, cache, N, stride, Hq=Hq, Hkv=Hkv)
    finally:
        attn.set_option("prefill_key_halves", 0)
    assert np.array_equal(run_prefill(attn, gpu, qkv, cache, N, stride, Hq=Hq, Hkv=Hkv), got)
    assert_close(got.reshape(N, -1)[rows].reshape(-1), exp, 2e-3, 1e-2, f"{Hq}/{Hkv} N={N}")
