"""Flash-Decode on the GPU vs the oracle.

* The reference's own known-answer test (test_causal_attention.cpp:152-228):
  closed-form inputs, head_dim {32, 128}, kv_heads {1, 2, 4}, lengths
  {1, 12, 13, 37, 257}, padded odd strides, output guards; tolerance 2e-3/2e-3.
* SmolLM3 shapes (16 query heads, 4 KV heads, D 128) at L up to 65536 with
  N(0,1) inputs and sentinel cache rows past L: |a - e| <= 2e-3 + 1e-2 |e|
  against the fp64 oracle.
* The result must not depend on the split plan; the workspace is only written
  inside the reference-sized capacity; graph nodes re-planned by
  update_causal_attention_decode_node replay bit-identically to eager launches.
"""
import numpy as np
import pytest
import torch

import oracle
from helpers import assert_close

pytestmark = pytest.mark.gpu

GUARD = np.float16(-123.0).view(np.uint16)


def dev(a, device):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.float16)).to(device)


def host(t):
    return t.detach().cpu().numpy().view(np.uint16)


def workspace(attn, device, Hq, L, D, guard_floats=64):
    """Reference-sized workspace (Hq*ceil(L/12) states) inside larger buffers
    whose tails are NaN canaries."""
    states = attn.decode_workspace_states(Hq, L)
    po = torch.full((states * D + guard_floats,), float("nan"), device=device)
    pm = torch.full((states + guard_floats,), float("nan"), device=device)
    ps = torch.full((states + guard_floats,), float("nan"), device=device)
    return po, pm, ps, states


def check_workspace_tails(ws, D):
    po, pm, ps, states = ws
    assert torch.isnan(po[states * D:]).all()
    assert torch.isnan(pm[states:]).all()
    assert torch.isnan(ps[states:]).all()


def run_decode(attn, device, q, k, v, L, Hq, Hkv, D, kv_stride=0, out_offset=1):
    q_dim = Hq * D
    dq, dk, dv = dev(q, device), dev(k, device), dev(v, device)
    out = torch.from_numpy(np.full(q_dim + 2 * out_offset, GUARD, dtype=np.uint16)
                           .view(np.float16)).to(device)
    ws = workspace(attn, device, Hq, L, D)
    attn.decode(dq, dk, dv, out.data_ptr() + 2 * out_offset, ws[0], ws[1], ws[2], 1, L, L - 1,
                Hq, Hkv, D, 0, kv_stride)
    torch.cuda.synchronize()
    got = host(out)
    assert np.all(got[:out_offset] == GUARD) and np.all(got[out_offset + q_dim:] == GUARD)
    check_workspace_tails(ws, D)
    return got[out_offset:out_offset + q_dim]


@pytest.mark.parametrize("head_dim", [32, 128])
@pytest.mark.parametrize("kv_heads", [1, 2, 4])
def test_reference_flash_decode_kat(attn, gpu, golden, head_dim, kv_heads):
    g = golden("kat_flash_decode.npz")
    heads = 4
    for length in (1, 12, 13, 37, 257):
        for padded in (0, 1):
            print(f"[case] KAT D={head_dim} kv={kv_heads} len={length} pad={padded}", flush=True)
            stride = kv_heads * head_dim + (17 if padded else 0)
            q, k, v = oracle.kat_inputs(heads, head_dim, kv_heads, length, stride)
            got = run_decode(attn, gpu, q, k, v, length, heads, kv_heads, head_dim,
                             kv_stride=stride if padded else 0)
            key = f"d{head_dim}_kv{kv_heads}_len{length}_pad{padded}"
            assert_close(got, g[key + "_expected"], 2e-3, 2e-3, key)


def smol_inputs(L, seed, cap_extra=2, sigma=1.0):
    Hq, Hkv, D = 16, 4, 128
    rng = np.random.default_rng(seed)
    q = (rng.standard_normal(Hq * D) * sigma).astype(np.float16).view(np.uint16)
    k = np.full((L + cap_extra) * Hkv * D, np.float16(123.0).view(np.uint16), dtype=np.uint16)
    v = k.copy()
    k[:L * Hkv * D] = (rng.standard_normal(L * Hkv * D) * sigma).astype(np.float16).view(np.uint16)
    v[:L * Hkv * D] = (rng.standard_normal(L * Hkv * D) * sigma).astype(np.float16).view(np.uint16)
    return q, k, v


def expected(q, k, v, L, Hq=16, Hkv=4, D=128):
    _, e32 = oracle.attention(q, k, v, 1, Hq, Hkv, D, Hq * D, Hkv * D, L, L - 1, causal=False)
    return e32.reshape(-1)


@pytest.mark.parametrize("L", [1, 2, 12, 13, 127, 128, 129, 254, 255, 1000, 3072, 4096, 4097,
                               12288, 12289, 16384, 20480, 20481, 32768, 32769, 65536])
def test_decode_smollm3_vs_oracle(attn, gpu, L):
    # the plan boundaries among them: 64-key chunks taken by one wave (4096)
    # against LDS-DMA chunks (4097), one against two KV heads per workgroup
    # (12288 / 12289), 160-key minimum chunks (12289 .. 20480) against 128
    # splits (20481), an odd chunk with three batches for one wave (32769)
    print(f"[case] decode L={L} plan={attn.decode_plan(L, 16, 4, 128)}", flush=True)
    q, k, v = smol_inputs(L, seed=3)
    got = run_decode(attn, gpu, q, k, v, L, 16, 4, 128)
    assert_close(got, expected(q, k, v, L), 2e-3, 1e-2, f"L={L}")


def test_decode_golden_fixtures(attn, gpu, golden):
    g = golden("attention.npz")
    for case in ("decode_a", "decode_b", "decode_c"):
        q, k, v, e = (g[f"{case}_{x}"] for x in ("q", "k", "v", "expected"))
        _, Hq, D = q.shape
        L, Hkv, _ = k.shape
        print(f"[case] decode golden {case} L={L} Hq={Hq} Hkv={Hkv} D={D}", flush=True)
        got = run_decode(attn, gpu, q.reshape(-1), k.reshape(-1), v.reshape(-1), L, Hq, Hkv, D)
        assert_close(got, e.reshape(-1), 2e-3, 2e-3, case)


@pytest.mark.parametrize("splits", [1, 2, 3, 7, 64, 256])
def test_decode_independent_of_split_plan(attn, gpu, splits):
    L = 20000
    q, k, v = smol_inputs(L, seed=9)
    e = expected(q, k, v, L)
    attn.set_option("decode_splits", splits)
    try:
        print(f"[case] decode L={L} splits={splits} plan={attn.decode_plan(L, 16, 4, 128)}",
              flush=True)
        got = run_decode(attn, gpu, q, k, v, L, 16, 4, 128)
    finally:
        attn.set_option("decode_splits", 0)
    assert_close(got, e, 2e-3, 1e-2, f"splits={splits}")


@pytest.mark.parametrize("hpw", [1, 2, 4])
def test_decode_heads_per_workgroup(attn, gpu, hpw):
    """Every split-kernel variant (1, 2 or 4 KV heads per workgroup) gives the
    oracle's result on SmolLM3 shapes."""
    L = 20001
    q, k, v = smol_inputs(L, seed=14)
    e = expected(q, k, v, L)
    attn.set_option("decode_heads_per_workgroup", hpw)
    try:
        plan = attn.decode_plan(L, 16, 4, 128)
        print(f"[case] decode hpw={hpw} plan={plan}", flush=True)
        assert attn.decode_hpw(plan["path"]) == hpw
        got = run_decode(attn, gpu, q, k, v, L, 16, 4, 128)
    finally:
        attn.set_option("decode_heads_per_workgroup", 0)
    assert_close(got, e, 2e-3, 1e-2, f"hpw={hpw}")


@pytest.mark.parametrize("L,hpw", [(37, 1), (254, 0), (4095, 0), (20001, 2), (20001, 4),
                                   (70001, 0)])
def test_decode_k_paths_bitidentical(attn, gpu, L, hpw):
    """K read through LDS-DMA in whole rows (decode_kdma=2) and K loaded into
    registers in the MFMA layout (decode_kdma=1) feed the same values to the
    same MFMAs: the outputs are bit-identical, and within tolerance of the
    oracle, with sentinel rows past L and chunks ending inside a batch."""
    q, k, v = smol_inputs(L, seed=15 + L % 7)
    e = expected(q, k, v, L)
    outs = {}
    attn.set_option("decode_heads_per_workgroup", hpw)
    try:
        for mode in (1, 2):
            attn.set_option("decode_kdma", mode)
            print(f"[case] decode L={L} hpw={hpw} kdma={mode} "
                  f"plan={attn.decode_plan(L, 16, 4, 128)}", flush=True)
            outs[mode] = run_decode(attn, gpu, q, k, v, L, 16, 4, 128)
    finally:
        attn.set_option("decode_kdma", 0)
        attn.set_option("decode_heads_per_workgroup", 0)
    assert np.array_equal(outs[1], outs[2])
    assert_close(outs[2], e, 2e-3, 1e-2, f"L={L} kdma")


def test_decode_forced_generic(attn, gpu):
    L = 5000
    q, k, v = smol_inputs(L, seed=10)
    e = expected(q, k, v, L)
    for opt, val in (("decode_force_generic", 1),):
        attn.set_option(opt, val)
        try:
            print(f"[case] decode {opt}={val} plan={attn.decode_plan(L, 16, 4, 128)}", flush=True)
            got = run_decode(attn, gpu, q, k, v, L, 16, 4, 128)
        finally:
            attn.set_option(opt, 0)
        assert_close(got, e, 2e-3, 1e-2, opt)


@pytest.mark.parametrize("Hq,Hkv", [(16, 16), (8, 1), (32, 2), (12, 4)])
def test_decode_other_group_sizes(attn, gpu, Hq, Hkv):
    L, D = 3000, 128
    rng = np.random.default_rng(Hq * 100 + Hkv)
    q = rng.standard_normal(Hq * D).astype(np.float16).view(np.uint16)
    k = rng.standard_normal(L * Hkv * D).astype(np.float16).view(np.uint16)
    v = rng.standard_normal(L * Hkv * D).astype(np.float16).view(np.uint16)
    print(f"[case] decode Hq={Hq} Hkv={Hkv} plan={attn.decode_plan(L, Hq, Hkv, D)}", flush=True)
    got = run_decode(attn, gpu, q, k, v, L, Hq, Hkv, D)
    assert_close(got, expected(q, k, v, L, Hq, Hkv, D), 2e-3, 1e-2, f"{Hq}/{Hkv}")


@pytest.mark.parametrize("L", [1, 20, 32, 33, 100, 254, 255, 383, 384, 385])
def test_decode_whole_context_plans(attn, gpu, L):
    """Up to 384 keys one workgroup per KV head takes the whole context (K
    through LDS-DMA, or straight into registers with decode_kdma = 1) and its
    fold writes the output (one kernel): within tolerance of the oracle, as
    is the two-kernel plan of the same inputs (option decode_whole_max_keys
    = -1), and the plan reports one split."""
    q, k, v = smol_inputs(L, seed=300 + L)
    plan = attn.decode_plan(L, 16, 4, 128)
    assert (plan["nsplit"] == 1 and plan["nstate"] == 1) == (L <= 384), plan
    print(f"[case] decode whole-context L={L} plan={plan}", flush=True)
    e = expected(q, k, v, L)
    got = run_decode(attn, gpu, q, k, v, L, 16, 4, 128)
    assert_close(got, e, 2e-3, 1e-2, f"whole L={L}")
    attn.set_option("decode_kdma", 1)
    try:
        reg = run_decode(attn, gpu, q, k, v, L, 16, 4, 128)
    finally:
        attn.set_option("decode_kdma", 0)
    assert np.array_equal(reg, got), "K paths differ"
    attn.set_option("decode_whole_max_keys", -1)
    try:
        assert attn.decode_plan(L, 16, 4, 128)["nsplit"] > 1 or L <= 16
        two = run_decode(attn, gpu, q, k, v, L, 16, 4, 128)
    finally:
        attn.set_option("decode_whole_max_keys", 0)
    assert_close(two, e, 2e-3, 1e-2, f"two kernels L={L}")


def test_decode_closed_forms(attn, gpu):
    # one key: the output is V[0] bit for bit; identical keys: the mean of V
    q, k, v = smol_inputs(1, seed=11)
    got = run_decode(attn, gpu, q, k, v, 1, 16, 4, 128)
    vv = v[:512].reshape(4, 128)
    assert np.array_equal(got.reshape(16, 128), np.repeat(vv, 4, axis=0))
    L = 777
    q, k, v = smol_inputs(L, seed=12)
    k[:L * 512] = np.tile(k[:512], L)
    got = run_decode(attn, gpu, q, k, v, L, 16, 4, 128)
    mean = v[:L * 512].view(np.float16).astype(np.float64).reshape(L, 4, 128).mean(axis=0)
    assert_close(got, np.repeat(mean, 4, axis=0).reshape(-1), 2e-3, 2e-3, "mean of V")


def test_decode_graph_node_update(attn, gpu):
    """model_inference.hpp:96-126: capture once, then patch kv_len with
    update_causal_attention_decode_node / update_merge_attention_decode_node
    and replay.  Each replay equals an eager launch bit for bit and the oracle
    within tolerance; eager work runs between replays."""
    import ctypes

    from attn_mi355x import hipgraph
    Lmax = 40000
    q, k, v = smol_inputs(Lmax, seed=13)
    dq, dk, dv = dev(q, gpu), dev(k, gpu), dev(v, gpu)
    states = attn.decode_workspace_states(16, Lmax)
    po = torch.empty(states * 128, device=gpu)
    pm = torch.empty(states, device=gpu)
    ps = torch.empty(states, device=gpu)
    out_g = torch.empty(2048, dtype=torch.float16, device=gpu)
    out_e = torch.empty(2048, dtype=torch.float16, device=gpu)
    po2, pm2, ps2 = po.clone(), pm.clone(), ps.clone()
    stream = torch.cuda.Stream()
    sp = stream.cuda_stream
    L0 = 100
    anode, mnode = ctypes.c_void_p(), ctypes.c_void_p()
    with torch.cuda.stream(stream):
        hipgraph.begin_capture(sp)
        rc = attn.lib().attn_decode(dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                                    out_g.data_ptr(), po.data_ptr(), pm.data_ptr(), ps.data_ptr(),
                                    1, L0, L0 - 1, 16, 4, 128, 3072, 512, sp,
                                    ctypes.byref(anode), ctypes.byref(mnode))
        assert rc == 0
        graph, exe = hipgraph.end_capture(sp)
    try:
        for L in (100, 101, 254, 4096, 4097, 33000, 39999, 100):
            assert attn.lib().attn_update_decode_node(exe, anode, L) == 0
            assert attn.lib().attn_update_merge_node(exe, mnode, L) == 0
            for rep in range(2):
                out_g.fill_(0.0)
                torch.cuda.synchronize()
                hipgraph.launch(exe, sp)
                hipgraph.synchronize(sp)
                attn.decode(dq, dk, dv, out_e, po2, pm2, ps2, 1, L, L - 1, 16, 4, 128, 0, 512)
                torch.cuda.synchronize()
                print(f"[case] decode graph L={L} replay {rep}", flush=True)
                assert np.array_equal(host(out_g), host(out_e)), (L, rep)
            assert_close(host(out_g), expected(q, k, v, L), 2e-3, 1e-2, f"graph L={L}")
    finally:
        hipgraph.destroy(graph, exe)


def test_graph_node_records(attn, gpu):
    """The updaters patch nodes from the records made at capture: a RoPE /
    append node and a decode pair captured into one graph are recorded (three
    records), patches from the records and patches that read every node back
    (option graph_node_records = 1, the reference's way) give bit-identical
    replays, equal to eager launches, and the records are dropped when the
    graph and its executable graph are destroyed."""
    import ctypes
    import time

    from attn_mi355x import hipgraph
    lib = attn.lib()
    Lmax = 9000
    q, k, v = smol_inputs(Lmax, seed=17)
    rng = np.random.default_rng(17)
    kn = rng.standard_normal(512).astype(np.float16).view(np.uint16)
    vn = rng.standard_normal(512).astype(np.float16).view(np.uint16)
    cos, sin = attn.rope_tables(Lmax, 128, 5e4)
    dcos, dsin = cos.reshape(-1).to(gpu), sin.reshape(-1).to(gpu)
    dq0, dk, dv = dev(q, gpu), dev(k, gpu), dev(v, gpu)
    dkn, dvn = dev(kn, gpu), dev(vn, gpu)
    states = attn.decode_workspace_states(16, Lmax)
    po, pm, ps = (torch.empty(states * 128, device=gpu), torch.empty(states, device=gpu),
                  torch.empty(states, device=gpu))
    dq = dq0.clone()
    out_g = torch.empty(2048, dtype=torch.float16, device=gpu)
    before = lib.attn_graph_node_records()
    stream = torch.cuda.Stream()
    sp = stream.cuda_stream
    anode, mnode = ctypes.c_void_p(), ctypes.c_void_p()
    L0 = 300
    with torch.cuda.stream(stream):
        hipgraph.begin_capture(sp)
        assert lib.attn_rope_store_kv(dq.data_ptr(), dkn.data_ptr(), dvn.data_ptr(), dk.data_ptr(),
                                      dv.data_ptr(), dcos.data_ptr(), dsin.data_ptr(), 1, 16, 4,
                                      128, 0, 0, L0 - 1, 1, sp) == 0
        rnode = hipgraph.last_captured_node(sp)
        assert lib.attn_decode(dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), out_g.data_ptr(),
                               po.data_ptr(), pm.data_ptr(), ps.data_ptr(), 1, L0, L0 - 1, 16, 4,
                               128, 0, 0, sp, ctypes.byref(anode), ctypes.byref(mnode)) == 0
        graph, exe = hipgraph.end_capture(sp)
    destroyed = False
    try:
        assert lib.attn_graph_node_records() == before + 3
        outs = {}
        for rec in (0, 1):
            attn.set_option("graph_node_records", rec)
            try:
                for L in (L0, 301, 4096, 8999, 301):
                    assert lib.attn_update_rope_node(exe, rnode, L - 1, 1) == 0
                    assert lib.attn_update_decode_node(exe, anode, L) == 0
                    assert lib.attn_update_merge_node(exe, mnode, L) == 0
                    dq.copy_(dq0)
                    torch.cuda.synchronize()
                    hipgraph.launch(exe, sp)
                    hipgraph.synchronize(sp)
                    print(f"[case] node records={rec} L={L}", flush=True)
                    outs.setdefault(L, []).append(host(out_g))
            finally:
                attn.set_option("graph_node_records", 0)
        for L, (a, b, *rest) in outs.items():
            assert np.array_equal(a, b), L
            for c in rest:
                assert np.array_equal(a, c), L
        # eager equivalent of the last replay (L = 301)
        dq.copy_(dq0)
        out_e = torch.empty(2048, dtype=torch.float16, device=gpu)
        attn.rope_store_kv(dq, dkn, dvn, dk, dv, dcos, dsin, 1, 16, 4, 128, 0, 0, 300, True)
        attn.decode(dq, dk, dv, out_e, po, pm, ps, 1, 301, 300, 16, 4, 128, 0, 0)
        torch.cuda.synchronize()
        assert np.array_equal(host(out_e), outs[301][-1])
        hipgraph.destroy(graph, exe)
        destroyed = True
        deadline = time.monotonic() + 5.0
        while lib.attn_graph_node_records() != before and time.monotonic() < deadline:
            time.sleep(0.01)
        assert lib.attn_graph_node_records() == before
    finally:
        if not destroyed:
            hipgraph.destroy(graph, exe)


@pytest.mark.parametrize("Hq,Hkv,hpw,L0", [(16, 2, 0, 50), (8, 1, 0, 50), (16, 4, 4, 50),
                                          (16, 4, 0, 19999)])
def test_decode_graph_node_update_other_paths(attn, gpu, Hq, Hkv, hpw, L0):
    """The node patchers re-plan every split-kernel variant (4, 2 or 1 KV
    heads per workgroup), including a change of variant with the context
    length (one KV head per workgroup up to 12288 keys, two above when Hkv is
    even), in both directions: replays equal eager launches bit for bit."""
    import ctypes

    from attn_mi355x import hipgraph
    D, Lmax = 128, 20000
    rng = np.random.default_rng(Hq * 10 + Hkv)
    q = rng.standard_normal(Hq * D).astype(np.float16).view(np.uint16)
    k = rng.standard_normal(Lmax * Hkv * D).astype(np.float16).view(np.uint16)
    v = rng.standard_normal(Lmax * Hkv * D).astype(np.float16).view(np.uint16)
    dq, dk, dv = dev(q, gpu), dev(k, gpu), dev(v, gpu)
    states = attn.decode_workspace_states(Hq, Lmax)
    po, pm, ps = (torch.empty(states * D, device=gpu), torch.empty(states, device=gpu),
                  torch.empty(states, device=gpu))
    po2, pm2, ps2 = po.clone(), pm.clone(), ps.clone()
    out_g = torch.empty(Hq * D, dtype=torch.float16, device=gpu)
    out_e = torch.empty(Hq * D, dtype=torch.float16, device=gpu)
    attn.set_option("decode_heads_per_workgroup", hpw)
    for L, expect_hpw in ((Lmax, 4 if hpw == 4 else (2 if Hkv % 2 == 0 else 1)),
                          (12288, 4 if hpw == 4 else 1), (12289, 4 if hpw == 4 else
                                                          (2 if Hkv % 2 == 0 else 1))):
        assert attn.decode_hpw(attn.decode_plan(L, Hq, Hkv, D)["path"]) == expect_hpw, L
    stream = torch.cuda.Stream()
    sp = stream.cuda_stream
    anode, mnode = ctypes.c_void_p(), ctypes.c_void_p()
    with torch.cuda.stream(stream):
        hipgraph.begin_capture(sp)
        rc = attn.lib().attn_decode(dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), out_g.data_ptr(),
                                    po.data_ptr(), pm.data_ptr(), ps.data_ptr(), 1, L0, L0 - 1, Hq,
                                    Hkv, D, 0, 0, sp, ctypes.byref(anode), ctypes.byref(mnode))
        assert rc == 0
        graph, exe = hipgraph.end_capture(sp)
    try:
        for L in (L0, 777, 4096, 12288, 12289, 19999, 50):
            assert attn.lib().attn_update_decode_node(exe, anode, L) == 0
            assert attn.lib().attn_update_merge_node(exe, mnode, L) == 0
            hipgraph.launch(exe, sp)
            hipgraph.synchronize(sp)
            attn.decode(dq, dk, dv, out_e, po2, pm2, ps2, 1, L, L - 1, Hq, Hkv, D)
            torch.cuda.synchronize()
            print(f"[case] decode graph Hq={Hq} Hkv={Hkv} L={L}", flush=True)
            assert np.array_equal(host(out_g), host(out_e)), (Hq, Hkv, L)
            assert_close(host(out_g), expected(q, k, v, L, Hq, Hkv, D), 2e-3, 1e-2,
                         f"graph {Hq}/{Hkv} L={L}")
    finally:
        hipgraph.destroy(graph, exe)
        attn.set_option("decode_heads_per_workgroup", 0)


@pytest.mark.parametrize("L", [100003, 131072])
def test_decode_long_contexts(attn, gpu, L):
    """Past C3's longest length, including an odd one: the split plan caps the
    split count and grows the chunk; still the oracle's result."""
    q, k, v = smol_inputs(L, seed=15)
    print(f"[case] decode L={L} plan={attn.decode_plan(L, 16, 4, 128)}", flush=True)
    got = run_decode(attn, gpu, q, k, v, L, 16, 4, 128)
    assert_close(got, expected(q, k, v, L), 2e-3, 1e-2, f"L={L}")


def test_decode_mfma_padded_kv_stride(attn, gpu):
    """A padded cache row (kv_stride 576, a multiple of 8) stays on the MFMA
    split path; rows past L hold sentinels."""
    L, Hq, Hkv, D, kvs = 5000, 16, 4, 128, 576
    rng = np.random.default_rng(16)
    q = rng.standard_normal(Hq * D).astype(np.float16).view(np.uint16)
    k = np.full((L + 2) * kvs, np.float16(123.0).view(np.uint16), dtype=np.uint16)
    v = k.copy()
    for buf in (k, v):
        rows = buf.reshape(L + 2, kvs)
        rows[:L, :Hkv * D] = rng.standard_normal((L, Hkv * D)).astype(np.float16).view(np.uint16)
    plan = attn.decode_plan(L, Hq, Hkv, D, kvs)
    print(f"[case] decode padded kv_stride={kvs} plan={plan}", flush=True)
    assert plan["path"] != 0
    got = run_decode(attn, gpu, q, k, v, L, Hq, Hkv, D, kv_stride=kvs)
    _, e32 = oracle.attention(q, k, v, 1, Hq, Hkv, D, Hq * D, kvs, L, L - 1, causal=False)
    assert_close(got, e32.reshape(-1), 2e-3, 1e-2, "padded kv_stride")


def test_decode_back_to_back_on_one_workspace(attn, gpu):
    """Calls queued back to back on one stream and one workspace, alternating
    inputs and lengths (so the partial states land at shifting places and
    split counts), each give their own oracle result: no call reads another's
    states."""
    Hq, Hkv, D = 16, 4, 128
    Ls = (32768, 5000, 32768, 777, 20001, 32768)
    inputs = {L: smol_inputs(L, seed=30 + i) for i, L in enumerate(sorted(set(Ls)))}
    dev_in = {L: tuple(dev(x, gpu) for x in inputs[L]) for L in inputs}
    po, pm, ps = attn.decode_workspace(Hq, max(Ls), D, device=gpu)
    outs = [torch.empty(Hq * D, dtype=torch.float16, device=gpu) for _ in range(3 * len(Ls))]
    for rep in range(3):
        for i, L in enumerate(Ls):
            dq, dk, dv = dev_in[L]
            attn.decode(dq, dk, dv, outs[rep * len(Ls) + i], po, pm, ps, 1, L, L - 1, Hq, Hkv, D,
                        0, 0)
    torch.cuda.synchronize()
    exp = {L: expected(*inputs[L], L) for L in inputs}
    for rep in range(3):
        for i, L in enumerate(Ls):
            print(f"[case] back-to-back rep={rep} L={L}", flush=True)
            got = host(outs[rep * len(Ls) + i])
            assert_close(got, exp[L], 2e-3, 1e-2, f"rep={rep} L={L}")
            if rep:
                assert np.array_equal(got, host(outs[i])), (rep, L)
