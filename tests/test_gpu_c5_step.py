"""Config C5 at its full shape: one decode token through all 36 layers of a
SmolLM3-3B-shaped KV cache ([36][K|V][32769][4 x 128] fp16, token-major,
kv_cache.hpp:20-34), RoPE on three layers of every four and NoPE on every 4th
(model_inference.hpp:358), the new token appended at position 32768 and
Flash-Decode over kv_len = 32769.

The step is captured as the engine captures it (model_inference.hpp:96-101,
361-387: per layer launch_rope_and_store_kv, then the decode's split and merge
kernels) and replayed once.  For every layer: the appended K row (rotated or
not) and V row, and q left rotated in place, equal the oracle's RoPE + append
bit for bit; the attention output is within the north-star tolerance of the
fp64 oracle over the layer's whole cache.  The same step issued through the
fused entry point (attn_rope_store_kv_decode, two kernels per layer) leaves
identical bits."""
import numpy as np
import pytest
import torch

import oracle
from helpers import assert_close

pytestmark = pytest.mark.gpu

LAYERS, HQ, HKV, D = 36, 16, 4, 128
Q_DIM, KV_DIM = HQ * D, HKV * D
QKV = Q_DIM + 2 * KV_DIM
POS = 32768            # the decoded token's position
L = POS + 1            # kv_len
S = L                  # cache capacity (max_seq_len)
SENT = 123.0


def test_c5_full_step_every_layer_vs_oracle(attn, gpu):
    from attn_mi355x import hipgraph
    lib = attn.lib()
    layer_elems = 2 * S * KV_DIM
    cache = torch.empty(LAYERS * layer_elems, dtype=torch.float16, device=gpu)
    g = torch.Generator(device=gpu)
    for layer in range(LAYERS):
        g.manual_seed(500 + layer)
        base = layer * layer_elems
        cache[base:base + layer_elems].normal_(generator=g)
        # the row the step must write holds a sentinel
        for half in range(2):
            row = base + half * S * KV_DIM + POS * KV_DIM
            cache[row:row + KV_DIM] = SENT
    g.manual_seed(499)
    qkv0 = torch.randn(LAYERS * QKV, generator=g, device=gpu).to(torch.float16)
    cache_fused = cache.clone()
    qkv_graph, qkv_fused = qkv0.clone(), qkv0.clone()
    cos, sin = attn.rope_tables(S, D, 5.0e6)
    dcos, dsin = cos.to(gpu), sin.to(gpu)
    out_graph = torch.empty(LAYERS * Q_DIM, dtype=torch.float16, device=gpu)
    out_fused = torch.empty_like(out_graph)
    po, pm, ps = attn.decode_workspace(HQ, L, D, device=gpu)
    e = 2  # bytes per element

    def ptrs(c, qkv, layer):
        kc = c.data_ptr() + e * layer * layer_elems
        vc = kc + e * S * KV_DIM
        row = qkv.data_ptr() + e * layer * QKV
        return row, row + e * Q_DIM, row + e * (Q_DIM + KV_DIM), kc, vc

    stream = torch.cuda.Stream()
    sp = stream.cuda_stream
    with torch.cuda.stream(stream):
        hipgraph.begin_capture(sp)
        for layer in range(LAYERS):
            q, k, v, kc, vc = ptrs(cache, qkv_graph, layer)
            apply = 1 if (layer + 1) % 4 != 0 else 0
            assert lib.attn_rope_store_kv(q, k, v, kc, vc, dcos.data_ptr(), dsin.data_ptr(), 1,
                                          HQ, HKV, D, QKV, QKV, POS, apply, sp) == 0
            assert lib.attn_decode(q, kc, vc, out_graph.data_ptr() + e * layer * Q_DIM,
                                   po.data_ptr(), pm.data_ptr(), ps.data_ptr(), 1, L, POS, HQ,
                                   HKV, D, QKV, KV_DIM, sp, None, None) == 0
        graph, exe = hipgraph.end_capture(sp)
        hipgraph.launch(exe, sp)
        hipgraph.synchronize(sp)
        hipgraph.destroy(graph, exe)
        for layer in range(LAYERS):
            q, k, v, kc, vc = ptrs(cache_fused, qkv_fused, layer)
            apply = 1 if (layer + 1) % 4 != 0 else 0
            assert lib.attn_rope_store_kv_decode(
                q, k, v, kc, vc, dcos.data_ptr(), dsin.data_ptr(),
                out_fused.data_ptr() + e * layer * Q_DIM, po.data_ptr(), pm.data_ptr(),
                ps.data_ptr(), L, POS, HQ, HKV, D, 0, apply, sp, None, None) == 0
        torch.cuda.synchronize()
    print("[case] C5 step captured, replayed and issued fused", flush=True)
    assert torch.equal(out_graph.view(torch.int16), out_fused.view(torch.int16))
    assert torch.equal(qkv_graph.view(torch.int16), qkv_fused.view(torch.int16))

    qkv_h = qkv0.cpu().numpy().view(np.uint16)
    qrot_h = qkv_graph.cpu().numpy().view(np.uint16)
    out_h = out_graph.cpu().numpy().view(np.uint16)
    ocos, osin = oracle.rope_tables(S, D, 5.0e6)
    for layer in range(LAYERS):
        base = layer * layer_elems
        kv_h = cache[base:base + layer_elems].cpu().numpy().view(np.uint16)
        kv_f = cache_fused[base:base + layer_elems].cpu().numpy().view(np.uint16)
        assert np.array_equal(kv_h, kv_f), layer
        k_h = kv_h[:S * KV_DIM].copy()
        v_h = kv_h[S * KV_DIM:].copy()
        # the oracle's RoPE + append of this layer's token into copies whose
        # row POS still holds the sentinel
        k_o, v_o = k_h.copy(), v_h.copy()
        k_o[POS * KV_DIM:L * KV_DIM] = np.float16(SENT).view(np.uint16)
        v_o[POS * KV_DIM:L * KV_DIM] = np.float16(SENT).view(np.uint16)
        row = qkv_h[layer * QKV:(layer + 1) * QKV].copy()
        q_o = row[:Q_DIM].copy()
        k_new = row[Q_DIM:Q_DIM + KV_DIM].copy()
        v_new = row[Q_DIM + KV_DIM:].copy()
        apply = (layer + 1) % 4 != 0
        oracle.rope_store_kv(q_o, k_new, v_new, k_o, v_o, ocos, osin, 1, HQ, HKV, D, Q_DIM,
                             KV_DIM, POS, apply)
        print(f"[case] C5 layer {layer} apply={int(apply)}", flush=True)
        assert np.array_equal(k_h, k_o), f"K rows, layer {layer}"
        assert np.array_equal(v_h, v_o), f"V rows, layer {layer}"
        assert np.array_equal(qrot_h[layer * QKV:layer * QKV + Q_DIM], q_o), f"q, layer {layer}"
        _, exp = oracle.attention(q_o, k_h, v_h, 1, HQ, HKV, D, Q_DIM, KV_DIM, L, POS,
                                  causal=False)
        assert_close(out_h[layer * Q_DIM:(layer + 1) * Q_DIM], exp.reshape(-1), 2e-3, 1e-2,
                     f"attention output, layer {layer}")
