"""Fused RoPE + KV append on the GPU vs the CPU oracle: bit-exact for every
byte of the source buffer and the cache (rotation values, copies, indexing,
untouched rows and layers).  Mirrors tests/test_rope.cpp:92-195 of the
reference (interleaved/packed x rotate/NoPE x start_pos, 2-layer cache with
sentinel rows) on seeded synthetic inputs."""
import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

SENTINEL = np.float16(-123.0).view(np.uint16)


def dev(a, device):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.float16)).to(device)


def host(t):
    return t.detach().cpu().numpy().view(np.uint16)


def run_case(attn, device, N, Hq, Hkv, D, start_pos, rotate, interleaved, theta=5.0e6,
             extra_q_stride=0, layers=2, layer=1, in_place_k=False):
    q_dim, kv_dim = Hq * D, Hkv * D
    S = start_pos + N + 2
    rng = np.random.default_rng(1000 * N + 10 * start_pos + int(rotate) + D)
    cos, sin = oracle.rope_tables(S, D, theta)
    dcos, dsin = dev(cos, device), dev(sin, device)
    if interleaved:
        stride = q_dim + 2 * kv_dim + extra_q_stride
        src = rng.standard_normal(N * stride).astype(np.float16).view(np.uint16)
        q_off, k_off, v_off = 0, q_dim, q_dim + kv_dim
        q_stride = k_stride = stride
    else:
        src = rng.standard_normal(N * (q_dim + 2 * kv_dim)).astype(np.float16).view(np.uint16)
        q_off, k_off, v_off = 0, N * q_dim, N * (q_dim + kv_dim)
        q_stride, k_stride = q_dim, kv_dim
    cache = np.full(layers * 2 * S * kv_dim, SENTINEL, dtype=np.uint16)
    kc_off = layer * 2 * S * kv_dim
    vc_off = kc_off + S * kv_dim

    d_src, d_cache = dev(src, device), dev(cache, device)
    base, cbase = d_src.data_ptr(), d_cache.data_ptr()
    if in_place_k:
        attn.rope(base + 2 * q_off, base + 2 * k_off, dcos, dsin, N, Hq, Hkv, D, q_stride,
                  k_stride, start_pos)
    else:
        attn.rope_store_kv(base + 2 * q_off, base + 2 * k_off, base + 2 * v_off,
                           cbase + 2 * kc_off, cbase + 2 * vc_off, dcos, dsin, N, Hq, Hkv, D,
                           q_stride, k_stride, start_pos, rotate)
    torch.cuda.synchronize()

    exp_src, exp_cache = src.copy(), cache.copy()
    # the oracle works on flat views of the same layout
    q_view = exp_src[q_off:]
    k_view = exp_src[k_off:]
    v_view = exp_src[v_off:]
    if in_place_k:
        oracle.rope_store_kv(q_view, k_view, None, None, None, cos, sin, N, Hq, Hkv, D,
                             q_stride, k_stride, start_pos, True)
    else:
        kc_view = exp_cache[kc_off:]
        vc_view = exp_cache[vc_off:]
        oracle.rope_store_kv(q_view, k_view, v_view, kc_view, vc_view, cos, sin, N, Hq, Hkv, D,
                             q_stride, k_stride, start_pos, rotate)
    got_src, got_cache = host(d_src), host(d_cache)
    assert np.array_equal(got_src, exp_src), "source buffer (Q in place / K,V unchanged)"
    assert np.array_equal(got_cache, exp_cache), "KV cache (rows, layers, sentinels)"
    return got_src, got_cache


@pytest.mark.parametrize("N", [1, 7, 254])
@pytest.mark.parametrize("start_pos", [0, 2])
@pytest.mark.parametrize("rotate", [True, False])
@pytest.mark.parametrize("interleaved", [True, False])
def test_rope_store_kv_engine_shapes(attn, gpu, N, start_pos, rotate, interleaved):
    print(f"[case] rope N={N} start={start_pos} rotate={rotate} interleaved={interleaved}",
          flush=True)
    run_case(attn, gpu, N, 16, 4, 128, start_pos, rotate, interleaved)


def test_rope_store_kv_prefill_8192(attn, gpu):
    print("[case] rope N=8192 interleaved rotate", flush=True)
    run_case(attn, gpu, 8192, 16, 4, 128, 0, True, True, layers=1, layer=0)


def test_rope_store_kv_decode_position_32768(attn, gpu):
    # C5: one token appended at position 32768 (cache S = 32770 here)
    for rotate in (True, False):
        print(f"[case] rope decode start=32768 rotate={rotate}", flush=True)
        run_case(attn, gpu, 1, 16, 4, 128, 32768, rotate, True, layers=1, layer=0)


def test_rope_store_kv_table_end(attn, gpu):
    # the last rows of a 131072-position table: a 7-token append ending at
    # position 131071 (fp32 angles of large positions, bit-exact vs the oracle)
    for rotate in (True, False):
        print(f"[case] rope start=131065 rotate={rotate}", flush=True)
        run_case(attn, gpu, 7, 16, 4, 128, 131065, rotate, True, layers=1, layer=0)


def test_launch_rope_in_place(attn, gpu):
    # launch_rope: K rotated in place, no cache (rope.hip.cpp:198-205,
    # test_qkv_gemm.cpp:91-94 interleaved strides)
    for interleaved in (True, False):
        print(f"[case] launch_rope interleaved={interleaved}", flush=True)
        run_case(attn, gpu, 33, 16, 4, 128, 0, True, interleaved, in_place_k=True)


@pytest.mark.parametrize("D,Hq,Hkv,extra", [(128, 16, 4, 3), (64, 8, 2, 0), (32, 4, 1, 5),
                                             (96, 6, 3, 0)])
def test_rope_generic_path(attn, gpu, D, Hq, Hkv, extra):
    # unaligned strides and head_dim not a multiple of 16 take the scalar kernel
    print(f"[case] rope generic D={D} Hq={Hq} Hkv={Hkv} extra={extra}", flush=True)
    run_case(attn, gpu, 37, Hq, Hkv, D, 3, True, True, theta=1.0e4, extra_q_stride=extra)
    run_case(attn, gpu, 37, Hq, Hkv, D, 3, False, True, theta=1.0e4, extra_q_stride=extra)


def test_rope_graph_node_update(attn, gpu):
    """Capture one decode-step RoPE/append (model_inference.hpp:358-368), then
    patch start_pos/apply with update_rope_and_store_kv_node and replay: every
    replay equals an eager launch at that position, bit for bit."""
    from attn_mi355x import hipgraph
    Hq, Hkv, D, S = 16, 4, 128, 64
    q_dim, kv_dim, stride = 2048, 512, 3072
    rng = np.random.default_rng(5)
    cos, sin = oracle.rope_tables(S, D, 5.0e6)
    dcos, dsin = dev(cos, gpu), dev(sin, gpu)
    src0 = rng.standard_normal(stride).astype(np.float16).view(np.uint16)
    d_src = dev(src0, gpu)
    d_cache = torch.full((2 * S * kv_dim,), -123.0, dtype=torch.float16, device=gpu)
    e_src = dev(src0, gpu)
    e_cache = d_cache.clone()
    stream = torch.cuda.Stream()
    sp = stream.cuda_stream
    base, cb = d_src.data_ptr(), d_cache.data_ptr()
    with torch.cuda.stream(stream):
        hipgraph.begin_capture(sp)
        attn.rope_store_kv(base, base + 2 * q_dim, base + 2 * (q_dim + kv_dim), cb,
                           cb + 2 * S * kv_dim, dcos, dsin, 1, Hq, Hkv, D, stride, stride, 0,
                           True, stream=sp)
        node = hipgraph.last_captured_node(sp)
        graph, exe = hipgraph.end_capture(sp)
    eb, ecb = e_src.data_ptr(), e_cache.data_ptr()
    try:
        for pos, rotate in ((5, True), (6, False), (40, True), (62, True), (0, True)):
            assert attn.lib().attn_update_rope_node(exe, node, pos, 1 if rotate else 0) == 0
            # fresh unrotated Q for this step in both buffers
            d_src.copy_(dev(src0, gpu))
            e_src.copy_(dev(src0, gpu))
            torch.cuda.synchronize()
            hipgraph.launch(exe, sp)
            hipgraph.synchronize(sp)
            attn.rope_store_kv(eb, eb + 2 * q_dim, eb + 2 * (q_dim + kv_dim), ecb,
                               ecb + 2 * S * kv_dim, dcos, dsin, 1, Hq, Hkv, D, stride, stride,
                               pos, rotate)
            torch.cuda.synchronize()
            assert np.array_equal(host(d_src), host(e_src)), pos
            assert np.array_equal(host(d_cache), host(e_cache)), pos
    finally:
        hipgraph.destroy(graph, exe)
