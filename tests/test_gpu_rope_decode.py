"""RoPE + KV append + Flash-Decode of one decode token as the decode's two
kernels (attn_rope_store_kv_decode; no reference counterpart).

The reference engine issues launch_rope_and_store_kv then
launch_causal_attention_decode per layer and token (model_inference.hpp:96-126).
The fused entry point must leave exactly the memory state of that pair: q
rotated in place, cache row start_pos holding K rotated and V copied (every
other row, sentinels included, untouched), and the same attention output, bit
for bit; graph replays patched by attn_update_rope_decode_nodes must equal
eager calls.  The pair itself is checked against the oracle elsewhere
(test_gpu_rope.py, test_gpu_decode.py); here the output is also bounded by the
fp64 oracle applied to the pair's memory state."""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from helpers import assert_close

pytestmark = pytest.mark.gpu

HQ, HKV, D = 16, 4, 128
Q_DIM, KV_DIM = HQ * D, HKV * D
SENT = np.float16(123.0).view(np.uint16)


def dev(a, device):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.float16)).to(device)


def host(t):
    return t.detach().cpu().numpy().view(np.uint16)


def inputs(L, start_pos, seed):
    """q, new k/v row, cache [S][KV_DIM] x 2 with rows < L random except the
    new token's row (sentinel: the call must write it), rows >= L sentinel."""
    rng = np.random.default_rng(seed)
    S = max(L, start_pos + 1) + 2

    def rnd(n):
        return rng.standard_normal(n).astype(np.float16).view(np.uint16)

    q, k, v = rnd(Q_DIM), rnd(KV_DIM), rnd(KV_DIM)
    cache = np.full(2 * S * KV_DIM, SENT, dtype=np.uint16)
    for half in range(2):
        rows = cache[half * S * KV_DIM:(half + 1) * S * KV_DIM].reshape(S, KV_DIM)
        rows[:L] = rnd(L * KV_DIM).reshape(L, KV_DIM)
        rows[start_pos] = SENT
    cos, sin = oracle.rope_tables(S, D, 5.0e6)
    return q, k, v, cache, cos, sin, S


class State:
    """Device copies of one input set plus output and workspace."""

    def __init__(self, attn, device, L, q, k, v, cache, cos, sin, S):
        self.q, self.k, self.v = dev(q, device), dev(k, device), dev(v, device)
        self.cache = dev(cache, device)
        self.kc = self.cache.data_ptr()
        self.vc = self.kc + 2 * S * KV_DIM
        self.cos, self.sin = dev(cos, device), dev(sin, device)
        self.out = torch.full((Q_DIM,), float("nan"), dtype=torch.float16, device=device)
        states = attn.decode_workspace_states(HQ, L)
        self.po = torch.empty(states * D, device=device)
        self.pm = torch.empty(states, device=device)
        self.ps = torch.empty(states, device=device)

    def snapshot(self):
        torch.cuda.synchronize()
        return host(self.q), host(self.cache), host(self.out)


def two_launches(attn, st, L, start_pos, apply):
    attn.rope_store_kv(st.q, st.k, st.v, st.kc, st.vc, st.cos, st.sin, 1, HQ, HKV, D, 0, 0,
                       start_pos, apply)
    attn.decode(st.q, st.kc, st.vc, st.out, st.po, st.pm, st.ps, 1, L, start_pos, HQ, HKV, D, 0,
                KV_DIM)


def fused(attn, st, L, start_pos, apply, stream=None, nodes=None):
    attn.rope_store_kv_decode(st.q, st.k, st.v, st.kc, st.vc, st.cos, st.sin, st.out, st.po,
                              st.pm, st.ps, L, start_pos, HQ, HKV, D, apply, stream=stream,
                              nodes=nodes)


@pytest.mark.parametrize("L,start_pos,apply,hpw", [
    (32769, 32768, True, 0), (254, 253, True, 0), (1, 0, True, 0), (254, 253, False, 0),
    (5000, 100, True, 0), (4096, 4095, True, 1), (4096, 4095, True, 4), (65536, 65535, False, 4),
    (300, 0, True, 0)])
def test_fused_equals_rope_then_decode(attn, gpu, L, start_pos, apply, hpw):
    print(f"[case] rope+decode L={L} pos={start_pos} apply={apply} hpw={hpw}", flush=True)
    q, k, v, cache, cos, sin, S = inputs(L, start_pos, seed=L + start_pos)
    attn.set_option("decode_heads_per_workgroup", hpw)
    try:
        a = State(attn, gpu, L, q, k, v, cache, cos, sin, S)
        two_launches(attn, a, L, start_pos, apply)
        ref = a.snapshot()
        b = State(attn, gpu, L, q, k, v, cache, cos, sin, S)
        fused(attn, b, L, start_pos, apply)
        got = b.snapshot()
    finally:
        attn.set_option("decode_heads_per_workgroup", 0)
    for x, y, what in zip(got, ref, ("q in place", "cache", "out")):
        assert np.array_equal(x, y), what
    # the pair's memory state through the fp64 oracle bounds the output
    qr, cr, _ = ref
    _, e32 = oracle.attention(qr, cr[:S * KV_DIM], cr[S * KV_DIM:], 1, HQ, HKV, D, Q_DIM, KV_DIM,
                              L, L - 1, causal=False)
    assert_close(got[2], e32.reshape(-1), 2e-3, 1e-2, "out vs oracle")


def test_fused_graph_replays_with_node_updates(attn, gpu):
    """Capture once, then per step patch kv_len / start_pos / apply_rotation
    with attn_update_rope_decode_nodes and replay; q is restored from a
    pristine copy between steps (the engine projects a fresh one).  Every
    replay equals an eager fused call on identical buffers bit for bit.
    Consecutive positions with the same state count and rotation switch
    leave the merge node unpatched (it reads the position the split kernel
    leaves in the workspace), so q must still be rotated at the new one."""
    from attn_mi355x import hipgraph
    Lmax = 40001
    q, k, v, cache, cos, sin, S = inputs(Lmax, Lmax - 1, seed=77)
    g = State(attn, gpu, Lmax, q, k, v, cache, cos, sin, S)
    e = State(attn, gpu, Lmax, q, k, v, cache, cos, sin, S)
    q0 = dev(q, gpu)
    stream = torch.cuda.Stream()
    sp = stream.cuda_stream
    nodes = []
    with torch.cuda.stream(stream):
        hipgraph.begin_capture(sp)
        fused(attn, g, 100, 99, True, stream=sp, nodes=nodes)
        graph, exe = hipgraph.end_capture(sp)
    try:
        for L, apply in ((100, True), (101, False), (254, True), (4097, True), (33000, False),
                         (33001, False), (33002, True), (33003, True), (33004, True),
                         (40001, True), (100, True)):
            assert attn.lib().attn_update_rope_decode_nodes(exe, nodes[0], nodes[1], L, L - 1,
                                                            1 if apply else 0) == 0
            for rep in range(2):
                g.q.copy_(q0)
                e.q.copy_(q0)
                g.out.fill_(0.0)
                torch.cuda.synchronize()
                hipgraph.launch(exe, sp)
                hipgraph.synchronize(sp)
                fused(attn, e, L, L - 1, apply)
                torch.cuda.synchronize()
                print(f"[case] rope+decode graph L={L} apply={apply} replay {rep}", flush=True)
                for x, y, what in zip(g.snapshot(), e.snapshot(), ("q", "cache", "out")):
                    assert np.array_equal(x, y), (L, rep, what)
    finally:
        hipgraph.destroy(graph, exe)


def test_fused_other_shapes_take_the_two_launches(attn, gpu):
    """Shapes the fused kernels do not serve (start_pos outside the decoded
    range, a padded kv_stride, head_dim 64): called eagerly they issue
    attn_rope_store_kv then attn_decode (the same bits as those two calls);
    asked for graph node handles they enqueue nothing and report
    hipErrorInvalidValue, since only the fused pair can be patched."""
    L = 64
    q, k, v, cache, cos, sin, S = inputs(L, L - 1, seed=5)
    lib = attn.lib()
    sp = torch.cuda.current_stream().cuda_stream
    args = lambda **kw: dict(dict(L=L, pos=L - 1, D=D, kvs=0, hq=HQ, hkv=HKV), **kw)

    def call(st, bad, nodes):
        an, mn = ctypes.c_void_p(), ctypes.c_void_p()
        return lib.attn_rope_store_kv_decode(
            st.q.data_ptr(), st.k.data_ptr(), st.v.data_ptr(), st.kc, st.vc, st.cos.data_ptr(),
            st.sin.data_ptr(), st.out.data_ptr(), st.po.data_ptr(), st.pm.data_ptr(),
            st.ps.data_ptr(), bad["L"], bad["pos"], bad["hq"], bad["hkv"], bad["D"], bad["kvs"], 1,
            sp, ctypes.byref(an) if nodes else None, ctypes.byref(mn) if nodes else None)

    for bad in (args(pos=L), args(kvs=KV_DIM + 8), args(D=64, kvs=0)):
        print(f"[case] fused rope+decode other shape {bad}", flush=True)
        st = State(attn, gpu, L, q, k, v, cache, cos, sin, S)
        before = st.snapshot()
        assert call(st, bad, nodes=True) == 1, bad  # hipErrorInvalidValue
        for x, y in zip(before, st.snapshot()):
            assert np.array_equal(x, y)
        assert call(st, bad, nodes=False) == 0, bad
        got = st.snapshot()
        ref = State(attn, gpu, L, q, k, v, cache, cos, sin, S)
        assert lib.attn_rope_store_kv(ref.q.data_ptr(), ref.k.data_ptr(), ref.v.data_ptr(),
                                      ref.kc, ref.vc, ref.cos.data_ptr(), ref.sin.data_ptr(), 1,
                                      bad["hq"], bad["hkv"], bad["D"], 0, 0, bad["pos"], 1,
                                      sp) == 0
        assert lib.attn_decode(ref.q.data_ptr(), ref.kc, ref.vc, ref.out.data_ptr(),
                               ref.po.data_ptr(), ref.pm.data_ptr(), ref.ps.data_ptr(), 1,
                               bad["L"], bad["pos"], bad["hq"], bad["hkv"], bad["D"], 0,
                               bad["kvs"], sp, None, None) == 0
        for x, y in zip(got, ref.snapshot()):
            assert np.array_equal(x, y), bad
