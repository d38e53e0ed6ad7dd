"""The attention output projection of a decode step on the GPU.

* launch_attention_out_projection_decode (kernels.hpp:179-187): the GEMV
  y = W x + beta y of matrix_vec_mul.hip.cpp:79-172 against the fp64 oracle
  (oracle.gemv_beta), beta 0 and 1, SmolLM3's 2048 x 2048 o_proj and odd
  shapes; guards around y.
* attn_decode_out_proj: by default the two launches (bit for bit); with the
  option decode_out_proj_fused = 1 the decode's merge fused into o_proj: the attention
  output it also writes against the fp64 oracle attention (north-star
  tolerance), y against the oracle GEMV applied to that same fp16 attention
  (at most one fp16 ulp: only the fp32 summation order differs), and against
  the two launches it replaces (attn_decode, attn_out_proj_decode); the
  counters of the workspace return to zero; repeated calls accumulate the
  residual; captured nodes patched to other kv_len replay bit-identically to
  eager calls; shapes off the fused path take the two launches.
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from helpers import assert_close, f16, ulp_diff

pytestmark = pytest.mark.gpu

GUARD = np.float16(123.0).view(np.uint16)


def dev(a, device):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.float16)).to(device)


def host(t):
    return t.detach().cpu().numpy().view(np.uint16)


def rnd(rng, n, scale=1.0):
    return (rng.standard_normal(n) * scale).astype(np.float16).view(np.uint16)


def guarded(y0, device):
    """y between two guard elements; returns (tensor, pointer to y)."""
    buf = dev(np.concatenate([[GUARD], y0, [GUARD]]).astype(np.uint16), device)
    return buf, buf.data_ptr() + 2


def unguard(buf):
    y = host(buf)
    assert y[0] == GUARD and y[-1] == GUARD, "write outside y"
    return y[1:-1]


@pytest.mark.parametrize("hidden,Hq,D", [(2048, 16, 128), (2000, 16, 128), (7, 3, 32),
                                         (37, 1, 2053), (5, 1, 0)])
@pytest.mark.parametrize("beta", [0.0, 1.0])
def test_out_proj_decode_vs_oracle(attn, gpu, hidden, Hq, D, beta):
    print(f"[case] o_proj hidden={hidden} Hq={Hq} D={D} beta={beta}", flush=True)
    in_dim = Hq * D
    rng = np.random.default_rng(hidden + in_dim + int(beta))
    w = rnd(rng, hidden * in_dim, 1.0 / np.sqrt(max(in_dim, 1))).reshape(hidden, in_dim)
    x = rnd(rng, in_dim)
    y0 = rnd(rng, hidden)
    buf, py = guarded(y0, gpu)
    dw, dx = dev(w, gpu), dev(x, gpu)
    attn.out_proj_decode(dx if in_dim else None, py, dw if in_dim else None, hidden, Hq, D, beta)
    torch.cuda.synchronize()
    y = unguard(buf)
    exp = oracle.gemv_beta(w, x, y0, beta)
    d = ulp_diff(y, exp)
    assert d.max() <= 1 and (d == 0).mean() > 0.99, (d.max(), (d == 0).mean())


def test_out_proj_decode_empty(attn, gpu):
    # hidden_size == 0 launches nothing, even with null pointers
    assert attn.lib().attn_out_proj_decode(None, None, None, 0, 16, 128, 1.0, None) == 0


@pytest.fixture
def fused(attn):
    """Selects the fused merge + o_proj kernel for the test's calls."""
    attn.set_option("decode_out_proj_fused", 1)
    yield
    attn.set_option("decode_out_proj_fused", 0)


def decode_inputs(L, Hq, Hkv, D, hidden, seed):
    rng = np.random.default_rng(seed)
    q = rnd(rng, Hq * D)
    k = np.full((L + 2) * Hkv * D, GUARD, dtype=np.uint16)
    v = k.copy()
    k[:L * Hkv * D] = rnd(rng, L * Hkv * D)
    v[:L * Hkv * D] = rnd(rng, L * Hkv * D)
    w = rnd(rng, hidden * Hq * D, 1.0 / np.sqrt(Hq * D)).reshape(hidden, Hq * D)
    y0 = rnd(rng, hidden)
    return q, k, v, w, y0


class Case:
    """Device buffers of one decode + o_proj step."""

    def __init__(self, attn, device, L, Hq, Hkv, D, hidden, seed=0, cap=None):
        self.attn, self.L, self.Hq, self.Hkv, self.D, self.hidden = attn, L, Hq, Hkv, D, hidden
        self.q, self.k, self.v, self.w, self.y0 = decode_inputs(cap or L, Hq, Hkv, D, hidden, seed)
        self.dq, self.dk, self.dv = dev(self.q, device), dev(self.k, device), dev(self.v, device)
        self.dw = dev(self.w, device)
        self.po, self.pm, self.ps = attn.decode_workspace(Hq, cap or L, D, device=device)
        self.ws = attn.decode_out_proj_workspace(Hq, hidden, device=device)
        self.device = device

    def fused(self, beta, L=None, y_buf=None, ws=True):
        L = L or self.L
        out = torch.empty(self.Hq * self.D, dtype=torch.float16, device=self.device)
        buf, py = y_buf if y_buf is not None else guarded(self.y0, self.device)
        self.attn.decode_out_proj(self.dq, self.dk, self.dv, out, self.po, self.pm, self.ps, L,
                                  self.Hq, self.Hkv, self.D, self.dw, py, self.hidden, beta,
                                  self.ws if ws else None)
        torch.cuda.synchronize()
        return unguard(buf), host(out)

    def two_launches(self, beta, L=None):
        L = L or self.L
        out = torch.empty(self.Hq * self.D, dtype=torch.float16, device=self.device)
        buf, py = guarded(self.y0, self.device)
        self.attn.decode(self.dq, self.dk, self.dv, out, self.po, self.pm, self.ps, 1, L, L - 1,
                         self.Hq, self.Hkv, self.D)
        self.attn.out_proj_decode(out, py, self.dw, self.hidden, self.Hq, self.D, beta)
        torch.cuda.synchronize()
        return unguard(buf), host(out)

    def oracle_attention(self, L=None):
        L = L or self.L
        kvd = self.Hkv * self.D
        _, e = oracle.attention(self.q, self.k, self.v, 1, self.Hq, self.Hkv, self.D,
                                self.Hq * self.D, kvd, L, L - 1, causal=False)
        return e.reshape(-1)

    def counters_zero(self):
        n_blocks = (self.hidden + 127) // 128
        tail = self.ws[self.ws.numel() - 4 * n_blocks:].cpu().numpy()
        return not tail.any()


def check_step(c, beta, y, attn_out, L=None):
    assert_close(attn_out, c.oracle_attention(L), 2e-3, 1e-2, "attention output")
    # the projection of the fp16 attention the kernel produced
    d = ulp_diff(y, oracle.gemv_beta(c.w, attn_out, c.y0, beta))
    assert d.max() <= 1 and (d == 0).mean() > 0.98, (d.max(), (d == 0).mean())


@pytest.mark.parametrize("L", [1, 7, 300, 4097, 12289, 32769])
@pytest.mark.parametrize("beta", [1.0, 0.0])
def test_decode_out_proj_smollm3(attn, gpu, fused, L, beta):
    print(f"[case] decode+o_proj SmolLM3 L={L} beta={beta}", flush=True)
    c = Case(attn, gpu, L, 16, 4, 128, 2048, seed=L)
    y, attn_out = c.fused(beta)
    assert c.counters_zero()
    check_step(c, beta, y, attn_out)
    # the pair of launches it replaces, with the same split plan (short
    # contexts would otherwise be decoded in one kernel, without fp16 partial
    # states): the same attention within fp32 merge-order rounding, the same
    # projection within the north-star tolerance
    attn.set_option("decode_whole_max_keys", -1)
    try:
        y2, attn2 = c.two_launches(beta)
    finally:
        attn.set_option("decode_whole_max_keys", 0)
    assert ulp_diff(attn_out, attn2).max() <= 1
    assert_close(y, y2, 2e-3, 1e-2, "fused vs two launches")


@pytest.mark.parametrize("Hq,Hkv,hidden,L", [(12, 4, 1000, 513), (8, 8, 100, 77),
                                             (16, 2, 2048, 2000), (32, 8, 4096, 999),
                                             (4, 1, 300, 40)])
def test_decode_out_proj_other_shapes(attn, gpu, fused, Hq, Hkv, hidden, L):
    """Row blocks that are partial or single, heads not a multiple of 8 (no
    XCD placement), other group sizes."""
    print(f"[case] decode+o_proj Hq={Hq} Hkv={Hkv} hidden={hidden} L={L}", flush=True)
    c = Case(attn, gpu, L, Hq, Hkv, 128, hidden, seed=Hq * 1000 + L)
    y, attn_out = c.fused(1.0)
    assert c.counters_zero()
    check_step(c, 1.0, y, attn_out)


@pytest.mark.parametrize("D,ws", [(64, True), (128, False)])
def test_decode_out_proj_two_launch_shapes(attn, gpu, fused, D, ws):
    """head_dim off the MFMA path, or no workspace: the two launches, bit for
    bit."""
    print(f"[case] decode+o_proj fallback D={D} workspace={ws}", flush=True)
    c = Case(attn, gpu, 300, 8, 2, D, 512, seed=D)
    y, attn_out = c.fused(1.0, ws=ws)
    y2, attn2 = c.two_launches(1.0)
    assert np.array_equal(y, y2) and np.array_equal(attn_out, attn2)
    check_step(c, 1.0, y, attn_out)


@pytest.mark.parametrize("L", [300, 32769])
def test_decode_out_proj_default_is_the_two_launches(attn, gpu, L):
    """Without the option the entry point issues attn_decode and
    attn_out_proj_decode: identical bits, counters untouched."""
    print(f"[case] decode+o_proj default L={L}", flush=True)
    c = Case(attn, gpu, L, 16, 4, 128, 2048, seed=L + 1)
    y, attn_out = c.fused(1.0)
    y2, attn2 = c.two_launches(1.0)
    assert np.array_equal(y, y2) and np.array_equal(attn_out, attn2)
    assert c.counters_zero()
    check_step(c, 1.0, y, attn_out)


def test_decode_out_proj_repeated_calls_accumulate(attn, gpu, fused):
    """Three calls on one workspace and one y (beta = 1): each adds W attn to
    the residual, so every call's counters must have been left at zero."""
    c = Case(attn, gpu, 4000, 16, 4, 128, 2048, seed=5)
    buf, py = guarded(c.y0, gpu)
    y_exp = c.y0
    for i, L in enumerate((4000, 3000, 17)):
        print(f"[case] repeated call {i} L={L}", flush=True)
        y, attn_out = c.fused(1.0, L=L, y_buf=(buf, py))
        assert c.counters_zero()
        y_exp = oracle.gemv_beta(c.w, attn_out, y_exp, 1.0)
        d = ulp_diff(y, y_exp)
        assert d.max() <= 1 and (d == 0).mean() > 0.98, (i, d.max())
        y_exp = y  # continue from the GPU's value


def test_decode_out_proj_graph_node_update(attn, gpu, fused):
    """Captured once (split node and fused merge + o_proj node), patched with
    attn_update_decode_node / attn_update_merge_node to other kv_len (across
    the plan's change of heads per workgroup) and replayed; each replay equals
    an eager call bit for bit, with eager work and synchronisation between."""
    from attn_mi355x import hipgraph
    Lmax = 20000
    c = Case(attn, gpu, Lmax, 16, 4, 128, 2048, seed=8)
    lib = attn.lib()
    out_g = torch.empty(2048, dtype=torch.float16, device=gpu)
    y_g = torch.empty(2048, dtype=torch.float16, device=gpu)
    y_init = dev(c.y0, gpu)
    stream = torch.cuda.Stream()
    sp = stream.cuda_stream
    anode, mnode = ctypes.c_void_p(), ctypes.c_void_p()
    ws_g = attn.decode_out_proj_workspace(16, 2048, device=gpu)
    po, pm, ps = attn.decode_workspace(16, Lmax, 128, device=gpu)
    L0 = 200
    with torch.cuda.stream(stream):
        hipgraph.begin_capture(sp)
        rc = lib.attn_decode_out_proj(c.dq.data_ptr(), c.dk.data_ptr(), c.dv.data_ptr(),
                                      out_g.data_ptr(), po.data_ptr(), pm.data_ptr(),
                                      ps.data_ptr(), L0, 16, 4, 128, 0, c.dw.data_ptr(),
                                      y_g.data_ptr(), 2048, 1.0, ws_g.data_ptr(), sp,
                                      ctypes.byref(anode), ctypes.byref(mnode))
        assert rc == 0
        graph, exe = hipgraph.end_capture(sp)
    try:
        for L in (200, 201, 4096, 12289, 19999, 200):
            assert lib.attn_update_decode_node(exe, anode, L) == 0
            assert lib.attn_update_merge_node(exe, mnode, L) == 0
            for rep in range(2):
                y_g.copy_(y_init)
                torch.cuda.synchronize()
                hipgraph.launch(exe, sp)
                hipgraph.synchronize(sp)
                y_e, attn_e = c.fused(1.0, L=L)
                print(f"[case] decode+o_proj graph L={L} replay {rep}", flush=True)
                assert np.array_equal(host(y_g), y_e), (L, rep)
                assert np.array_equal(host(out_g), attn_e), (L, rep)
            assert not ws_g[ws_g.numel() - 64:].cpu().numpy().any()
        check_step(c, 1.0, host(y_g), host(out_g), L=200)
    finally:
        hipgraph.destroy(graph, exe)
