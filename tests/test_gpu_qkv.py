"""Decode-step QKV projection on the GPU: the GEMV of launch_qkv_decode
(kernels.hpp:38-45) against the fp64 oracle, and the fused projection + RoPE +
KV append against the two launches it replaces (model_inference.hpp:354-369),
bit for bit.  The GEMV cases mirror tests/test_matrix_vec_mul.cpp:8-70 of the
reference (its shapes, closed-form inputs, guard elements and tolerance);
SmolLM3's 2048 -> 3072 projection runs on seeded random inputs."""
import numpy as np
import pytest
import torch

import oracle
from helpers import assert_close, f16, ulp_diff

pytestmark = pytest.mark.gpu

GUARD = np.float16(123.0).view(np.uint16)
SENTINEL = np.float16(-123.0).view(np.uint16)


def dev(a, device):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.float16)).to(device)


def host(t):
    return t.detach().cpu().numpy().view(np.uint16)


def reference_inputs(out_dim, in_dim):
    """test_matrix_vec_mul.cpp:21-24."""
    i = np.arange(out_dim * in_dim)
    w = (((i % 29) - 14) / 64.0).astype(np.float16).view(np.uint16).reshape(out_dim, in_dim)
    x = (((np.arange(in_dim) % 17) - 8) / 16.0).astype(np.float16).view(np.uint16)
    return w, x


def run_gemv(attn, device, w, x, offset=0):
    """W and x start `offset` elements into their buffers; y sits between two
    guard elements, its rows pre-filled with NaN (test_matrix_vec_mul.cpp:27-41)."""
    out_dim, in_dim = w.shape
    pad = np.zeros(offset, np.uint16), np.zeros(1, np.uint16)
    d_w = dev(np.concatenate([pad[0], w.ravel(), pad[1]]), device)
    d_x = dev(np.concatenate([pad[0], x, pad[1]]), device)
    y0 = np.full(out_dim + 2, np.float16(np.nan).view(np.uint16), dtype=np.uint16)
    y0[0] = y0[-1] = GUARD
    d_y = dev(y0, device)
    attn.qkv_decode(d_x.data_ptr() + 2 * offset, d_y.data_ptr() + 2, d_w.data_ptr() + 2 * offset,
                    in_dim, out_dim)
    torch.cuda.synchronize()
    y = host(d_y)
    assert y[0] == GUARD and y[-1] == GUARD, "write outside y"
    return y[1:-1]


REFERENCE_SHAPES = [(1, 1, 0), (7, 31, 0), (129, 129, 0), (37, 2048, 0), (19, 11008, 0),
                    (22016, 2048, 0), (2048, 2048, 0), (3072, 2048, 0), (3, 0, 0), (7, 8, 0),
                    (9, 2053, 0), (5, 2056, 0), (7, 4096, 0), (5, 2056, 1)]


@pytest.mark.parametrize("out_dim,in_dim,offset", REFERENCE_SHAPES)
def test_qkv_decode_reference_shapes(attn, gpu, out_dim, in_dim, offset):
    print(f"[case] gemv out={out_dim} in={in_dim} offset={offset}", flush=True)
    w, x = reference_inputs(out_dim, in_dim)
    y = run_gemv(attn, gpu, w, x, offset)
    exp = f16(w).astype(np.float64) @ f16(x).astype(np.float64)
    # the reference test's tolerance against fp64 (test_matrix_vec_mul.cpp:58)
    assert_close(y, exp, 1e-3, 1e-3, "GEMV vs fp64")
    assert ulp_diff(y, oracle.gemv(w, x)).max() <= 1


@pytest.mark.parametrize("out_dim,in_dim,offset", [(3072, 2048, 0), (3072, 2048, 3),
                                                   (1023, 2040, 0), (4, 520, 0)])
def test_qkv_decode_random_vs_oracle(attn, gpu, out_dim, in_dim, offset):
    """SmolLM3's projection (hidden 2048 -> (16 + 2*4) * 128) on random inputs,
    and the vector loop's tail and element-loop variants."""
    print(f"[case] gemv random out={out_dim} in={in_dim} offset={offset}", flush=True)
    rng = np.random.default_rng(out_dim + in_dim + offset)
    w = (rng.standard_normal((out_dim, in_dim)) / np.sqrt(in_dim)).astype(np.float16)
    x = rng.standard_normal(in_dim).astype(np.float16)
    w, x = w.view(np.uint16), x.view(np.uint16)
    y = run_gemv(attn, gpu, w, x, offset)
    exp = oracle.gemv(w, x)
    # fp16 outputs within 2e-3 abs / 1e-2 rel of the fp64 oracle; the fp32 sums
    # differ from it only in order, so at most one fp16 ulp and rarely at all
    assert_close(y, exp, 2e-3, 1e-2, "GEMV vs oracle")
    d = ulp_diff(y, exp)
    assert d.max() <= 1 and (d == 0).mean() > 0.99


def test_qkv_decode_empty(attn, gpu):
    # total_qkv_dim == 0 launches nothing, even with null pointers
    # (test_matrix_vec_mul.cpp:68-70)
    assert attn.lib().attn_qkv_decode(None, None, None, 2048, 0, None) == 0


def fused_case(attn, device, Hq, Hkv, D, hidden, start_pos, rotate, offset=0, seed=0):
    """Runs the fused kernel and the two-kernel sequence on the same inputs.
    Returns (fused y, fused cache, two-kernel y, two-kernel cache, inputs)."""
    q_dim, kv_dim = Hq * D, Hkv * D
    total = q_dim + 2 * kv_dim
    S = start_pos + 3
    rng = np.random.default_rng(seed + 17 * start_pos + D)
    w = (rng.standard_normal((total, hidden)) / np.sqrt(hidden)).astype(np.float16)
    x = rng.standard_normal(hidden).astype(np.float16)
    w, x = w.view(np.uint16), x.view(np.uint16)
    cos, sin = oracle.rope_tables(S, D, 5.0e6)
    dcos, dsin = dev(cos, device), dev(sin, device)
    d_w = dev(np.concatenate([np.zeros(offset, np.uint16), w.ravel()]), device)
    d_x = dev(np.concatenate([np.zeros(offset, np.uint16), x]), device)
    pw, px = d_w.data_ptr() + 2 * offset, d_x.data_ptr() + 2 * offset
    cache0 = np.full(2 * S * kv_dim, SENTINEL, dtype=np.uint16)
    outs = []
    for fused in (True, False):
        d_y = torch.empty(total, dtype=torch.float16, device=device)
        d_c = dev(cache0, device)
        y, kc, vc = d_y.data_ptr(), d_c.data_ptr(), d_c.data_ptr() + 2 * S * kv_dim
        if fused:
            attn.qkv_rope_store_kv_decode(px, y, pw, kc, vc, dcos, dsin, hidden, Hq, Hkv, D,
                                          start_pos, rotate)
        else:
            attn.qkv_decode(px, y, pw, hidden, total)
            attn.rope_store_kv(y, y + 2 * q_dim, y + 2 * (q_dim + kv_dim), kc, vc, dcos, dsin,
                               1, Hq, Hkv, D, total, total, start_pos, rotate)
        torch.cuda.synchronize()
        outs += [host(d_y), host(d_c)]
    return outs + [(w, x, cos, sin, cache0, S)]


@pytest.mark.parametrize("Hq,Hkv,D,hidden", [(16, 4, 128, 2048), (8, 2, 64, 1024),
                                             (4, 4, 32, 520), (2, 1, 128, 2053)])
@pytest.mark.parametrize("start_pos", [0, 5, 32767])
@pytest.mark.parametrize("rotate", [True, False])
def test_qkv_rope_store_kv_fused_bitexact(attn, gpu, Hq, Hkv, D, hidden, start_pos, rotate):
    """Fused == launch_qkv_decode + launch_rope_and_store_kv, bit for bit in y
    and in every cache element (rows written, sentinel rows untouched); and the
    oracle's RoPE applied to the GPU GEMV output gives the same bits."""
    print(f"[case] fused Hq={Hq} Hkv={Hkv} D={D} hidden={hidden} pos={start_pos} "
          f"rotate={rotate}", flush=True)
    fy, fc, ty, tc, (w, x, cos, sin, cache0, S) = fused_case(attn, gpu, Hq, Hkv, D, hidden,
                                                           start_pos, rotate)
    assert np.array_equal(fy, ty), "y"
    assert np.array_equal(fc, tc), "cache"
    # CPU check of the epilogue: oracle rope_store_kv on the GPU's own GEMV output
    q_dim, kv_dim = Hq * D, Hkv * D
    g = run_gemv(attn, gpu, w, x)
    q, k, v = g[:q_dim].copy(), g[q_dim:q_dim + kv_dim].copy(), g[q_dim + kv_dim:].copy()
    ec = cache0.copy()
    oracle.rope_store_kv(q, k, v, ec[:S * kv_dim], ec[S * kv_dim:], cos, sin, 1, Hq, Hkv, D,
                         q_dim, kv_dim, start_pos, rotate)
    assert np.array_equal(fy, np.concatenate([q, k, v])), "y vs GEMV + oracle RoPE"
    assert np.array_equal(fc, ec), "cache vs GEMV + oracle RoPE"
    # and the whole step against the all-oracle step (fp64 GEMV) within tolerance
    oc = cache0.copy()
    oy = oracle.qkv_rope_store_kv_decode(w, x, oc[:S * kv_dim], oc[S * kv_dim:], cos, sin, Hq,
                                         Hkv, D, start_pos, rotate)
    assert_close(fy, oy, 2e-3, 1e-2, "y vs oracle step")
    assert_close(fc, oc, 2e-3, 1e-2, "cache vs oracle step")


def test_qkv_rope_store_kv_fused_unaligned(attn, gpu):
    """x and W one element past 16-byte alignment take the element loop; the
    fused result still equals the two launches."""
    fy, fc, ty, tc, _ = fused_case(attn, gpu, 16, 4, 128, 2048, 9, True, offset=1)
    assert np.array_equal(fy, ty) and np.array_equal(fc, tc)


def test_qkv_rope_graph_node_update(attn, gpu):
    """Capture the fused node once, patch start_pos / apply_rotation per step
    with attn_update_qkv_rope_node, replay: each replay equals an eager fused
    launch at that position (y and cache), bit for bit."""
    from attn_mi355x import hipgraph
    Hq, Hkv, D, hidden, S = 16, 4, 128, 2048, 64
    q_dim, kv_dim = Hq * D, Hkv * D
    total = q_dim + 2 * kv_dim
    rng = np.random.default_rng(11)
    cos, sin = oracle.rope_tables(S, D, 5.0e6)
    dcos, dsin = dev(cos, gpu), dev(sin, gpu)
    d_w = dev((rng.standard_normal((total, hidden)) / 45.0).astype(np.float16).view(np.uint16),
              gpu)
    d_x = dev(rng.standard_normal(hidden).astype(np.float16).view(np.uint16), gpu)
    d_y = torch.empty(total, dtype=torch.float16, device=gpu)
    e_y = torch.empty_like(d_y)
    d_c = torch.full((2 * S * kv_dim,), -123.0, dtype=torch.float16, device=gpu)
    e_c = d_c.clone()
    stream = torch.cuda.Stream()
    sp = stream.cuda_stream
    cb, ecb = d_c.data_ptr(), e_c.data_ptr()
    with torch.cuda.stream(stream):
        hipgraph.begin_capture(sp)
        attn.qkv_rope_store_kv_decode(d_x, d_y, d_w, cb, cb + 2 * S * kv_dim, dcos, dsin, hidden,
                                      Hq, Hkv, D, 0, True, stream=sp)
        node = hipgraph.last_captured_node(sp)
        graph, exe = hipgraph.end_capture(sp)
    try:
        for pos, rotate in ((5, True), (6, False), (40, True), (63, True), (0, True)):
            assert attn.lib().attn_update_qkv_rope_node(exe, node, pos, 1 if rotate else 0) == 0
            hipgraph.launch(exe, sp)
            hipgraph.synchronize(sp)
            attn.qkv_rope_store_kv_decode(d_x, e_y, d_w, ecb, ecb + 2 * S * kv_dim, dcos, dsin,
                                          hidden, Hq, Hkv, D, pos, rotate)
            torch.cuda.synchronize()
            assert np.array_equal(host(d_y), host(e_y)), pos
            assert np.array_equal(host(d_c), host(e_c)), pos
        # a node of another kernel is refused
        assert attn.lib().attn_update_rope_node(exe, node, 1, 1) != 0
    finally:
        hipgraph.destroy(graph, exe)
