"""The library is stateless across calls (no global scratch, plans derived from
the arguments), so host threads driving their own streams and workspaces must
get exactly the results of the same calls issued one at a time.  The
reference engine drives one stream per process (model_inference.hpp:31); this
covers a server that runs several sequences side by side."""
import threading

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

HQ, HKV, D = 16, 4, 128
Q_DIM, KV_DIM, QKV = HQ * D, HKV * D, (HQ + 2 * HKV) * D


def make_job(attn, device, kind, seed):
    """Returns (inputs, run(stream) -> output tensor) for one kind of call."""
    g = torch.Generator(device="cpu").manual_seed(seed)

    def rnd(n, scale=1.0):
        return (torch.randn(n, generator=g) * scale).to(torch.float16).to(device)

    if kind == "decode":
        L = 3000 + 97 * seed
        q, kc, vc = rnd(Q_DIM), rnd((L + 1) * KV_DIM), rnd((L + 1) * KV_DIM)
        po, pm, ps = attn.decode_workspace(HQ, L, D, device=device)
        out = torch.empty(Q_DIM, dtype=torch.float16, device=device)

        def run(stream):
            attn.decode(q, kc, vc, out, po, pm, ps, 1, L, L - 1, HQ, HKV, D, QKV, KV_DIM,
                        stream=stream)
            return out
    elif kind == "prefill":
        N = 300 + 11 * seed
        qkv, kc, vc = rnd(N * QKV, 0.5), rnd(N * KV_DIM, 0.5), rnd(N * KV_DIM, 0.5)
        out = torch.empty(N * Q_DIM, dtype=torch.float16, device=device)

        def run(stream):
            attn.prefill(qkv, kc, vc, out, N, HQ, HKV, D, QKV, KV_DIM, stream=stream)
            return out
    else:  # fused decode QKV projection + RoPE + append
        S = 64
        x, w = rnd(2048), rnd(QKV * 2048, 1.0 / 45)
        cos, sin = attn.rope_tables(S, D, 5.0e6)
        dcos, dsin = cos.to(device), sin.to(device)
        y = torch.empty(QKV, dtype=torch.float16, device=device)
        cache = torch.zeros(2 * S * KV_DIM, dtype=torch.float16, device=device)
        pos = 7 + seed

        def run(stream):
            attn.qkv_rope_store_kv_decode(x, y, w, cache, cache.data_ptr() + 2 * S * KV_DIM,
                                          dcos, dsin, 2048, HQ, HKV, D, pos, True, stream=stream)
            return torch.cat([y, cache])
    return run


def test_threads_on_own_streams_match_serial(attn, gpu):
    kinds = ["decode", "prefill", "qkv", "decode", "prefill", "qkv"]
    jobs = [make_job(attn, gpu, k, i) for i, k in enumerate(kinds)]
    torch.cuda.synchronize()
    expected = []
    for run in jobs:  # one at a time on the default stream
        expected.append(run(None).clone())
        torch.cuda.synchronize()
    streams = [torch.cuda.Stream() for _ in jobs]
    results = [None] * len(jobs)
    errors = []
    barrier = threading.Barrier(len(jobs))

    def worker(i):
        try:
            barrier.wait()
            with torch.cuda.stream(streams[i]):
                for _ in range(20):
                    out = jobs[i](streams[i].cuda_stream)
                streams[i].synchronize()
                results[i] = out.clone()
                streams[i].synchronize()
        except Exception as e:  # reported below
            errors.append((i, repr(e)))

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(len(jobs))]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=60)
    assert not any(t.is_alive() for t in threads), "worker did not finish"
    assert not errors, errors
    torch.cuda.synchronize()
    for i, (r, e) in enumerate(zip(results, expected)):
        assert np.array_equal(r.cpu().numpy().view(np.uint16), e.cpu().numpy().view(np.uint16)), \
            (i, kinds[i])
