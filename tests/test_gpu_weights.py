"""A weights.bin in device memory feeding the attention path: the reference's
QKV test chain (tests/test_qkv_gemm.cpp:26-119) on a synthetic SmolLM3-shaped
file (hidden 2048, 16 x 128 query and 4 x 128 KV heads, two layers, small
vocabulary and MLP).  The reference runs the chain on real checkpoint
activations (tests/reference/*.bin), which need the SmolLM3 checkpoint and do
not exist here; this file is written by oracle/weights_file.py in the
exporter's format with seeded weights, and the expected values come from the
oracle: the fp64 GEMM on the weights read back from the file at the positions
the writer recorded, the oracle's RoPE, and the fp64-softmax attention.

Covered: the uploaded payload equals the file byte for byte; a layer's fused
QKV weight found through the library's layout is exactly the file's q_proj |
k_proj | v_proj (the GEMM on it equals the GEMM on those tensors uploaded
separately, bit for bit); GEMM -> RoPE -> prefill on the interleaved
[N][3072] output against the oracle; the same chain through the C++ headers
(MemoryMappedFile + Model, tests/cpp/test_model_weights.cpp) gives the same
bits; the decode step (fused QKV GEMV + RoPE + append, then Flash-Decode) on
a loaded layer against the oracle."""
import pathlib
import subprocess

import numpy as np
import pytest
import torch

import oracle
import weights_file as wf
from helpers import assert_close

pytestmark = pytest.mark.gpu

ROOT = pathlib.Path(__file__).resolve().parents[1]
CPP_BIN = ROOT / "tests" / "cpp" / "_build" / "test_model_weights"
CFG = dict(wf.SMOLLM3_3B, vocab_size=256, num_layers=2, intermediate_size=512, max_seq_len=512)
HQ, HKV, D, HIDDEN = 16, 4, 128, 2048
Q_DIM, KV_DIM = HQ * D, HKV * D
TOTAL = Q_DIM + 2 * KV_DIM


def dev(a, device):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.float16)).to(device)


def host(t):
    return t.detach().cpu().numpy().view(np.uint16)


@pytest.fixture(scope="module")
def model_file(tmp_path_factory):
    path = tmp_path_factory.mktemp("weights") / "weights.bin"
    base, where = wf.write(path, CFG, b'{"version": "1.0", "model": "synthetic"}', seed=11)
    return path, base, where


@pytest.fixture(scope="module")
def loaded(attn, gpu, model_file):
    path, _, _ = model_file
    return attn.ModelWeights(path, gpu)


def file_qkv(model_file, layer):
    path, base, where = model_file
    p = f"model.layers.{layer}.self_attn."
    return np.concatenate([wf.read_tensor(path, base, where, p + n + ".weight")
                           for n in ("q_proj", "k_proj", "v_proj")], axis=0)


def test_upload_equals_file_payload(loaded, model_file):
    path, base, _ = model_file
    payload = np.fromfile(path, dtype=np.uint16, offset=base)
    assert loaded.layout.weights_offset == base
    assert loaded.buffer.numel() == payload.size
    assert np.array_equal(host(loaded.buffer), payload)
    assert loaded.tokenizer_json == b'{"version": "1.0", "model": "synthetic"}'


def chain(attn, gpu, w_ptr, x, n):
    """GEMM -> RoPE (in place) -> prefill, as test_qkv_gemm.cpp:50-112."""
    d_x = dev(x, gpu)
    y = torch.empty(n * TOTAL, dtype=torch.float16, device=gpu)
    attn.qkv_gemm(d_x, y, w_ptr, n, HIDDEN, TOTAL)
    torch.cuda.synchronize()
    g = host(y)
    cos, sin = attn.rope_tables(CFG["max_seq_len"], D, CFG["rope_theta"])
    dcos, dsin = cos.to(gpu), sin.to(gpu)
    attn.rope(y, y.data_ptr() + 2 * Q_DIM, dcos, dsin, n, HQ, HKV, D, TOTAL, TOTAL)
    torch.cuda.synchronize()
    r = host(y)
    out = torch.empty(n * Q_DIM, dtype=torch.float16, device=gpu)
    attn.prefill(y, y.data_ptr() + 2 * Q_DIM, y.data_ptr() + 2 * (Q_DIM + KV_DIM), out, n, HQ,
                 HKV, D, TOTAL, TOTAL)
    torch.cuda.synchronize()
    return g, r, host(out), (cos.numpy().view(np.uint16), sin.numpy().view(np.uint16))


@pytest.mark.parametrize("layer,n", [(0, 254), (1, 254), (1, 64)])
def test_qkv_chain_on_loaded_weights(attn, gpu, loaded, model_file, layer, n):
    print(f"[case] weights chain layer={layer} n={n}", flush=True)
    rng = np.random.default_rng(100 + layer)
    x = rng.standard_normal((n, HIDDEN)).astype(np.float16).view(np.uint16)
    w = file_qkv(model_file, layer)
    qkv = loaded.qkv(layer)
    assert qkv.shape == (TOTAL, HIDDEN)
    g, r, out, (cos, sin) = chain(attn, gpu, qkv.data_ptr(), x, n)

    # the loaded pointer addresses exactly the file's q_proj | k_proj | v_proj
    d_w = dev(w, gpu)
    y2 = torch.empty(n * TOTAL, dtype=torch.float16, device=gpu)
    attn.qkv_gemm(dev(x, gpu), y2, d_w, n, HIDDEN, TOTAL)
    torch.cuda.synchronize()
    assert np.array_equal(g, host(y2)), "GEMM on loaded weights vs file tensors"

    # GEMM vs the fp64 oracle on the file's tensors
    exp = oracle.gemm(x, w)
    assert_close(g.reshape(n, TOTAL), exp, 2e-3, 1e-2, "QKV GEMM vs oracle")

    # RoPE on the GEMM output: bit-exact with the oracle's (rope.hip.cpp:44-58)
    er = g.copy()
    oracle.rope_store_kv(er, er[Q_DIM:], None, None, None, cos, sin, n, HQ, HKV, D, TOTAL, TOTAL,
                         0, True)
    assert np.array_equal(r, er), "RoPE vs oracle"

    # prefill attention on the interleaved buffer vs the fp64-softmax oracle
    _, e32 = oracle.attention(r, r[Q_DIM:], r[Q_DIM + KV_DIM:], n, HQ, HKV, D, TOTAL, TOTAL, n)
    assert_close(out, e32.reshape(-1), 2e-3, 1e-2, "prefill vs oracle")


@pytest.mark.parametrize("layer", [0, 1])
def test_cpp_model_chain(attn, gpu, loaded, model_file, tmp_path, layer):
    """The same chain through MemoryMappedFile + Model + the C++ launchers."""
    assert CPP_BIN.exists(), f"{CPP_BIN} not built: run __graft_entry__.build()"
    path, base, where = model_file
    n = 254
    rng = np.random.default_rng(100 + layer)
    x = rng.standard_normal((n, HIDDEN)).astype(np.float16).view(np.uint16)
    prefix = tmp_path / "chain"
    x.tofile(f"{prefix}.x")
    print(f"[case] C++ model chain layer={layer}", flush=True)
    r = subprocess.run([str(CPP_BIN), str(path), str(prefix), str(n), str(layer)],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    lines = r.stdout.splitlines()
    p = f"model.layers.{layer}.self_attn."
    expect = [where[p + t + ".weight"][0] // 2 for t in ("q_proj", "k_proj", "v_proj", "o_proj")]
    expect.append(where["lm_head.weight"][0] // 2)
    assert lines[0] == "offsets " + " ".join(map(str, expect))
    assert lines[1] == "tokenizer 40"
    assert lines[-1] == "done"
    g, rr, out, _ = chain(attn, gpu, loaded.qkv(layer).data_ptr(), x, n)
    for suffix, mine in (("qkv", g), ("rope", rr), ("attn", out)):
        theirs = np.fromfile(f"{prefix}.{suffix}", dtype=np.uint16)
        assert np.array_equal(theirs, mine), suffix


@pytest.mark.parametrize("layer,apply", [(0, True), (1, True), (1, False)])
def test_decode_step_on_loaded_weights(attn, gpu, loaded, model_file, layer, apply):
    """The engine's decode step on a loaded layer (model_inference.hpp:354-387):
    the QKV GEMV on block.q_proj with its RoPE + KV append fused
    (launch_qkv_rope_and_store_kv_decode), then Flash-Decode over the cache.
    The GEMV on the loaded pointer equals the GEMV on the file's tensors bit
    for bit; y and the new cache row equal the oracle's RoPE applied to that
    GEMV bit for bit and the all-oracle step within tolerance; the attention
    output is within tolerance of the fp64-softmax oracle."""
    pos, S = 300, 320
    print(f"[case] decode step layer={layer} apply={apply}", flush=True)
    rng = np.random.default_rng(200 + layer)
    x = rng.standard_normal(HIDDEN).astype(np.float16).view(np.uint16)
    cache = rng.standard_normal(2 * S * KV_DIM).astype(np.float16).view(np.uint16)
    cache[pos * KV_DIM:(pos + 1) * KV_DIM] = 0
    cache[(S + pos) * KV_DIM:(S + pos + 1) * KV_DIM] = 0
    w = file_qkv(model_file, layer)
    cos, sin = attn.rope_tables(CFG["max_seq_len"], D, CFG["rope_theta"])
    d_c = dev(cache, gpu)
    kc, vc = d_c.data_ptr(), d_c.data_ptr() + 2 * S * KV_DIM
    y = torch.empty(TOTAL, dtype=torch.float16, device=gpu)
    attn.qkv_rope_store_kv_decode(dev(x, gpu), y, loaded.qkv(layer), kc, vc, cos.to(gpu),
                                  sin.to(gpu), HIDDEN, HQ, HKV, D, pos, apply)
    torch.cuda.synchronize()
    got_y, got_c = host(y), host(d_c)

    g = torch.empty(TOTAL, dtype=torch.float16, device=gpu)
    attn.qkv_decode(dev(x, gpu), g, dev(w, gpu), HIDDEN, TOTAL)
    torch.cuda.synchronize()
    g = host(g)
    c16, s16 = cos.numpy().view(np.uint16), sin.numpy().view(np.uint16)
    q, k, v = g[:Q_DIM].copy(), g[Q_DIM:Q_DIM + KV_DIM].copy(), g[Q_DIM + KV_DIM:].copy()
    ec = cache.copy()
    oracle.rope_store_kv(q, k, v, ec[:S * KV_DIM], ec[S * KV_DIM:], c16, s16, 1, HQ, HKV, D,
                         Q_DIM, KV_DIM, pos, apply)
    assert np.array_equal(got_y, np.concatenate([q, g[Q_DIM:]])), "y vs GEMV + oracle RoPE"
    assert np.array_equal(got_c, ec), "cache vs GEMV + oracle RoPE"

    oc = cache.copy()
    oy = oracle.qkv_rope_store_kv_decode(w, x, oc[:S * KV_DIM], oc[S * KV_DIM:], c16, s16, HQ,
                                         HKV, D, pos, apply)
    assert_close(got_y, oy, 2e-3, 1e-2, "y vs oracle step")
    assert_close(got_c, oc, 2e-3, 1e-2, "cache vs oracle step")

    L = pos + 1
    out = torch.full((Q_DIM,), float("nan"), dtype=torch.float16, device=gpu)
    po, pm, ps = attn.decode_workspace(HQ, L, D, gpu)
    attn.decode(y, kc, vc, out, po, pm, ps, 1, L, pos, HQ, HKV, D, 0, KV_DIM)
    torch.cuda.synchronize()
    _, e32 = oracle.attention(got_y, got_c[:S * KV_DIM], got_c[S * KV_DIM:], 1, HQ, HKV, D, Q_DIM,
                              KV_DIM, L, L - 1, causal=False)
    assert_close(host(out), e32.reshape(-1), 2e-3, 1e-2, "decode vs oracle")
