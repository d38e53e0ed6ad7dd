"""Prefill QKV projection on the GPU: launch_qkv_gemm (kernels.hpp:29-36, the
rocBLAS product of qkv_gemm.hip.cpp:7-105) against the fp64 oracle GEMM, and
the fused projection + RoPE + KV append against the two launches it replaces
(model_inference.hpp:266-285), bit for bit.  Seeded synthetic inputs; the
reference's own QKV test (test_qkv_gemm.cpp) needs checkpoint fixtures that do
not exist here, so its shapes (SmolLM3: hidden 2048 -> 3072) are used with
random data."""
import numpy as np
import pytest
import torch

import oracle
from helpers import assert_close, ulp_diff

pytestmark = pytest.mark.gpu

GUARD = np.float16(123.0).view(np.uint16)
SENTINEL = np.float16(-123.0).view(np.uint16)
HQ, HKV, D, HIDDEN = 16, 4, 128, 2048
TOTAL = (HQ + 2 * HKV) * D


def dev(a, device):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.float16)).to(device)


def host(t):
    return t.detach().cpu().numpy().view(np.uint16)


def rand_inputs(M, N, K, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((M, K)).astype(np.float16).view(np.uint16)
    w = (rng.standard_normal((N, K)) / np.sqrt(max(K, 1))).astype(np.float16).view(np.uint16)
    return x, w


def run_gemm(attn, device, x, w, offset=0):
    """X and W start `offset` elements into their buffers; Y sits between two
    guard elements, pre-filled with NaN."""
    M, K = x.shape
    N = w.shape[0]
    pad = np.zeros(offset, np.uint16), np.zeros(1, np.uint16)
    d_x = dev(np.concatenate([pad[0], x.ravel(), pad[1]]), device)
    d_w = dev(np.concatenate([pad[0], w.ravel(), pad[1]]), device)
    y0 = np.full(M * N + 2, np.float16(np.nan).view(np.uint16), dtype=np.uint16)
    y0[0] = y0[-1] = GUARD
    d_y = dev(y0, device)
    attn.qkv_gemm(d_x.data_ptr() + 2 * offset, d_y.data_ptr() + 2, d_w.data_ptr() + 2 * offset,
                  M, K, N)
    torch.cuda.synchronize()
    y = host(d_y)
    assert y[0] == GUARD and y[-1] == GUARD, "write outside y"
    return y[1:-1].reshape(M, N)


def check_vs_oracle(y, x, w, rows=None):
    M, K = x.shape
    if rows is None and M * w.shape[0] * K > 4e8:
        # bounded oracle time: tile edges and a stride of the rows
        rows = np.unique(np.concatenate([[0, M - 1], np.arange(63, M, 64), np.arange(0, M, 9)]))
    exp = oracle.gemm(x if rows is None else x[rows], w)
    got = y if rows is None else y[rows]
    # fp16 outputs within 2e-3 abs / 1e-2 rel of the fp64 oracle; the fp32 sums
    # differ from it only in order and rounding, so nearly all elements are
    # bit-equal (near-zero sums of cancelling terms can differ by a few ulps)
    assert_close(got, exp, 2e-3, 1e-2, "GEMM vs oracle")
    d = ulp_diff(got, exp)
    big = np.abs(got.view(np.float16).astype(np.float32)) >= 0.25
    assert (d == 0).mean() > 0.99 and d[big].max(initial=0) <= 1, (d.max(), (d == 0).mean())


@pytest.mark.parametrize("M,N,K,offset", [
    (254, TOTAL, HIDDEN, 0),   # C2 prefill length (64 tokens per workgroup)
    (513, TOTAL, HIDDEN, 0),   # 128 tokens per workgroup, token tail
    (1500, 384, 256, 0),       # 256 tokens per workgroup, token tail, 3 feature tiles
    (300, 200, 128, 0),        # feature tail inside a tile
    (65, 1000, 64, 0),         # one k-stage; feature tiles not a multiple of 8
    (1, 128, 64, 0),
    (7, 33, 31, 0),            # K not a multiple of 64: element kernel
    (5, 40, 72, 1),            # unaligned X and W: element kernel
])
def test_qkv_gemm_vs_oracle(attn, gpu, M, N, K, offset):
    print(f"[case] gemm M={M} N={N} K={K} offset={offset}", flush=True)
    x, w = rand_inputs(M, N, K, M + N + K + offset)
    y = run_gemm(attn, gpu, x, w, offset)
    check_vs_oracle(y, x, w)


def test_qkv_gemm_empty_and_zero_k(attn, gpu):
    lib = attn.lib()
    # seq_len == 0 or total == 0 launches nothing, even with null pointers
    assert lib.attn_qkv_gemm(None, None, None, 0, 2048, 3072, None) == 0
    assert lib.attn_qkv_gemm(None, None, None, 8, 2048, 0, None) == 0
    # hidden == 0: an empty sum, y = 0 (rocBLAS with k = 0 and beta = 0)
    y = torch.full((3 * 10,), float("nan"), dtype=torch.float16, device=gpu)
    attn.qkv_gemm(None, y, None, 3, 0, 10)
    torch.cuda.synchronize()
    assert torch.all(y == 0)


def test_qkv_gemm_smollm3_8192(attn, gpu):
    """C4's projection: 8192 tokens x 2048 -> 3072.  Sampled rows (first,
    last, tile edges, random) against the oracle; every row against a torch
    fp32 product on the GPU."""
    M = 8192
    print(f"[case] gemm M={M} N={TOTAL} K={HIDDEN}", flush=True)
    x, w = rand_inputs(M, TOTAL, HIDDEN, 77)
    y = run_gemm(attn, gpu, x, w)
    rows = np.unique(np.concatenate([[0, 1, 255, 256, 4095, 4096, 8190, 8191],
                                     np.random.default_rng(1).integers(0, M, 40)]))
    check_vs_oracle(y, x, w, rows)
    ref = (dev(x, gpu).float() @ dev(w, gpu).float().t()).cpu().numpy()
    assert_close(y, ref, 2e-3, 1e-2, "GEMM vs torch fp32")


@pytest.mark.parametrize("tokens_per_wave", [32, 64, 128])
@pytest.mark.parametrize("M,N", [(700, TOTAL), (1100, 1280)])
def test_qkv_gemm_tile_variants_identical(attn, gpu, tokens_per_wave, M, N):
    """Every tile shape (64, 128 or 256 tokens x 128 features) sums each
    output in the same k order, so all variants give the same bits (and match
    the oracle)."""
    print(f"[case] gemm variants M={M} N={N} tpw={tokens_per_wave}", flush=True)
    x, w = rand_inputs(M, N, HIDDEN, 5)
    base = run_gemm(attn, gpu, x, w)
    try:
        attn.set_option("qkv_gemm_tokens_per_wave", tokens_per_wave)
        y = run_gemm(attn, gpu, x, w)
    finally:
        attn.set_option("qkv_gemm_tokens_per_wave", 0)
    assert np.array_equal(y, base)
    check_vs_oracle(y, x, w, np.arange(0, M, 7))


def fused_case(attn, device, M, start_pos, rotate, Hq=HQ, Hkv=HKV, Dh=D, K=HIDDEN, offset=0,
               seed=0):
    """Fused kernel and the two-kernel sequence on the same inputs; returns
    (fused y, fused cache, two-kernel y, two-kernel cache, inputs)."""
    q_dim, kv_dim = Hq * Dh, Hkv * Dh
    N = q_dim + 2 * kv_dim
    S = start_pos + M + 3
    x, w = rand_inputs(M, N, K, seed + 31 * start_pos + M)
    cos, sin = oracle.rope_tables(S, Dh, 5.0e6)
    dcos, dsin = dev(cos, device), dev(sin, device)
    pad = np.zeros(offset, np.uint16)
    d_x = dev(np.concatenate([pad, x.ravel()]), device)
    d_w = dev(np.concatenate([pad, w.ravel()]), device)
    px, pw = d_x.data_ptr() + 2 * offset, d_w.data_ptr() + 2 * offset
    cache0 = np.full(2 * S * kv_dim, SENTINEL, dtype=np.uint16)
    outs = []
    for fused in (True, False):
        d_y = torch.empty(M * N, dtype=torch.float16, device=device)
        d_c = dev(cache0, device)
        y, kc, vc = d_y.data_ptr(), d_c.data_ptr(), d_c.data_ptr() + 2 * S * kv_dim
        if fused:
            attn.qkv_gemm_rope_store_kv(px, y, pw, kc, vc, dcos, dsin, M, K, Hq, Hkv, Dh,
                                        start_pos, rotate)
        else:
            attn.qkv_gemm(px, y, pw, M, K, N)
            attn.rope_store_kv(y, y + 2 * q_dim, y + 2 * (q_dim + kv_dim), kc, vc, dcos, dsin, M,
                               Hq, Hkv, Dh, N, N, start_pos, rotate)
        torch.cuda.synchronize()
        outs += [host(d_y).reshape(M, N), host(d_c)]
    return outs + [(x, w, cos, sin, cache0, S)]


@pytest.mark.parametrize("M,start_pos,rotate", [(254, 0, True), (254, 0, False), (1000, 37, True),
                                                (3000, 5, True), (64, 32700, False),
                                                (8192, 0, True), (4100, 9, False)])
def test_qkv_gemm_rope_store_kv_fused_bitexact(attn, gpu, M, start_pos, rotate):
    """Fused == launch_qkv_gemm + launch_rope_and_store_kv bit for bit in Y
    and every cache element; the oracle's RoPE applied to the GPU GEMM output
    gives the same bits; the whole step is within tolerance of the all-oracle
    step (fp64 GEMM)."""
    print(f"[case] fused gemm M={M} pos={start_pos} rotate={rotate}", flush=True)
    fy, fc, ty, tc, (x, w, cos, sin, cache0, S) = fused_case(attn, gpu, M, start_pos, rotate)
    assert np.array_equal(fy, ty), "y"
    assert np.array_equal(fc, tc), "cache"
    q_dim, kv_dim = HQ * D, HKV * D
    g = ty if not rotate else run_gemm(attn, gpu, x, w)
    q = np.ascontiguousarray(g[:, :q_dim])
    k = np.ascontiguousarray(g[:, q_dim:q_dim + kv_dim])
    v = np.ascontiguousarray(g[:, q_dim + kv_dim:])
    ec = cache0.copy()
    oracle.rope_store_kv(q, k, v, ec[:S * kv_dim], ec[S * kv_dim:], cos, sin, M, HQ, HKV, D,
                         q_dim, kv_dim, start_pos, rotate)
    assert np.array_equal(fy, np.concatenate([q, k, v], axis=1)), "y vs GEMM + oracle RoPE"
    assert np.array_equal(fc, ec), "cache vs GEMM + oracle RoPE"
    if M <= 256:
        ox = oracle.gemm(x, w)
        oq = np.ascontiguousarray(ox[:, :q_dim])
        ok = np.ascontiguousarray(ox[:, q_dim:q_dim + kv_dim])
        ov = np.ascontiguousarray(ox[:, q_dim + kv_dim:])
        oc = cache0.copy()
        oracle.rope_store_kv(oq, ok, ov, oc[:S * kv_dim], oc[S * kv_dim:], cos, sin, M, HQ, HKV,
                             D, q_dim, kv_dim, start_pos, rotate)
        assert_close(fy, np.concatenate([oq, ok, ov], axis=1), 2e-3, 1e-2, "y vs oracle step")
        assert_close(fc, oc, 2e-3, 1e-2, "cache vs oracle step")


@pytest.mark.parametrize("Hq,Hkv,Dh,K,offset", [(8, 2, 64, 256, 0), (16, 4, 128, 2048, 1)])
def test_qkv_gemm_rope_store_kv_other_shapes(attn, gpu, Hq, Hkv, Dh, K, offset):
    """head_dim != 128 or unaligned operands take the two launches inside the
    same entry point: results identical to calling them."""
    fy, fc, ty, tc, _ = fused_case(attn, gpu, 130, 3, True, Hq, Hkv, Dh, K, offset)
    assert np.array_equal(fy, ty) and np.array_equal(fc, tc)


def test_qkv_fused_prefill_pipeline_matches_reference_order(attn, gpu):
    """Fused projection -> prefill attention equals the reference's order
    (GEMM, RoPE + append, prefill) bit for bit at C2's 254 tokens."""
    M, q_dim, kv_dim = 254, HQ * D, HKV * D
    fy, fc, ty, tc, (_, _, _, _, _, S) = fused_case(attn, gpu, M, 0, True)
    outs = []
    for y, c in ((fy, fc), (ty, tc)):
        d_y, d_c = dev(y, gpu), dev(c, gpu)
        out = torch.empty(M * q_dim, dtype=torch.float16, device=gpu)
        attn.prefill(d_y, d_c, d_c.data_ptr() + 2 * S * kv_dim, out, M, HQ, HKV, D, TOTAL,
                     kv_dim)
        torch.cuda.synchronize()
        outs.append(host(out))
    assert np.array_equal(outs[0], outs[1])


def with_wide(attn, mode, fn):
    attn.set_option("qkv_gemm_wide", mode)
    try:
        return fn()
    finally:
        attn.set_option("qkv_gemm_wide", 0)


@pytest.mark.parametrize("M,N,K", [(700, TOTAL, HIDDEN), (256, 384, 64), (1, 384, 128),
                                   (300, 1152, 512), (4100, TOTAL, HIDDEN)])
def test_qkv_gemm_wide_tile_identical(attn, gpu, M, N, K):
    """The 256 x 384 tile sums every output's k-chunks in the same order as
    the 256 x 128 tile: identical bits, and the oracle bounds both."""
    print(f"[case] gemm wide M={M} N={N} K={K}", flush=True)
    x, w = rand_inputs(M, N, K, 9 + M)
    narrow = with_wide(attn, 1, lambda: run_gemm(attn, gpu, x, w))
    wide = with_wide(attn, 2, lambda: run_gemm(attn, gpu, x, w))
    assert np.array_equal(wide, narrow)
    check_vs_oracle(wide, x, w, np.unique(np.r_[0, M - 1, np.arange(0, M, 13)]))


@pytest.mark.parametrize("M,start_pos,rotate", [(1000, 37, True), (300, 5, False),
                                                (8192, 0, True), (257, 32000, True)])
def test_qkv_gemm_wide_fused_identical(attn, gpu, M, start_pos, rotate):
    """The fused wide tile writes the bytes of the fused 256 x 128 tile (Y and
    every cache element, sentinel rows untouched)."""
    print(f"[case] fused gemm wide M={M} pos={start_pos} rotate={rotate}", flush=True)
    narrow = with_wide(attn, 1, lambda: fused_case(attn, gpu, M, start_pos, rotate))
    wide = with_wide(attn, 2, lambda: fused_case(attn, gpu, M, start_pos, rotate))
    for a_, b_, what in zip(wide[:4], narrow[:4], ("fused y", "fused cache", "two-step y",
                                                   "two-step cache")):
        assert np.array_equal(a_, b_), what
    assert np.array_equal(wide[0], wide[2]) and np.array_equal(wide[1], wide[3])
