#!/usr/bin/env python3
"""Benchmark of the MI355X attention hot path (one GPU).

Headline (BASELINE.json metric "decode-attn HBM GB/s (% of peak) @32K ctx;
prefill-attn TFLOPS @8K tokens"):
  value      = Flash-Decode HBM throughput at L = 32768 (config C3), one query
               token, 16 query heads / 4 KV heads / head_dim 128, algorithmic
               bytes 2048*L + 8192 per call, KV rotated over 8 buffers
               (8 x 67 MB > 256 MB Infinity Cache) so every call streams HBM.
               A "step" is one decode call over one KV buffer; the K timed
               steps are one HIP-graph replay of K captured calls (the
               engine's decode also replays a graph, model_inference.hpp:
               96-126), HIP events on the launch stream; after a 0.25 s device
               warm-up (streaming reads) the graph is replayed 15 times and
               the median replay gives ms_per_step (min / median / max in
               detail).
  prefill    = causal prefill TFLOPS at N = 8192 (config C4), algorithmic
               FLOPs 4096*N*(N+1): median of 60 launches each timed with its
               own HIP events, after 40 warm-up launches.
Also reported: every C3 length warm and cold, the same rotated K/V bytes read
by a plain streaming kernel (the ceiling a decode call can approach), C1/C2,
RoPE+append at 8192 tokens, the 36-layer attention-only decode step C5 as one
replayed graph and as the reference engine runs it (per token: every layer's
nodes patched through the C++ updaters, graph launch, synchronize), and CPU
baselines timed on this host: cpu_baseline is the reference's PyTorch CPU
attention (python/reference.py:61-96 restated with torch SDPA, fp16, all torch
threads) on a ~10 s sample of C3 decode calls; the fp64 C oracle (1 thread) is
in detail.  Inputs are seeded synthetic N(0, sigma) tensors.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick] [--no-cpu]
       python bench.py --profile   (eager launches for rocprofv3 counter passes)
       python bench.py --timeline  (per-segment decode timeline, instrumented library)
"""
from __future__ import annotations

import argparse
import json
import math
import os
import pathlib
import platform
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "llm-inference_amd" / "python"))

PEAK_HBM_GBS = 8000.0          # MI355X HBM3E, GB/s
PEAK_FP16_TFLOPS = 2500.0      # MI355X dense fp16 MFMA, TFLOP/s
HQ, HKV, D = 16, 4, 128
Q_DIM, KV_DIM, QKV = HQ * D, HKV * D, HQ * D + 2 * HKV * D
THETA = 5.0e6


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def decode_bytes(L):
    return 2 * L * HKV * D * 2 + 2 * HQ * D * 2


def prefill_flops(N):
    return 2 * HQ * D * N * (N + 1)


def rope_bytes(N, rotate=True):
    return (12544 if rotate else 4096) * N


HIDDEN = 2048  # SmolLM3-3B hidden size: the decode QKV projection is 2048 -> QKV


def qkv_bytes():
    """Algorithmic HBM bytes of one decode QKV GEMV: W, x and y once."""
    return 2 * (QKV * HIDDEN + HIDDEN + QKV)


def rand16(torch, n, seed, sigma=1.0, device="cuda"):
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return (torch.randn(n, generator=g, device=device) * sigma).to(torch.float16)


def time_graph(torch, A, hipgraph, launch_one, steps, warmup, stream, replays=7,
               before_replay=None):
    """Warm up with `warmup` eager launches, capture `steps` launches into one
    graph, replay it once untimed, then `replays` times inside event brackets
    on the launch stream, each bracketed by synchronizations (and preceded,
    outside the brackets, by `before_replay(stream)` when given).  Returns ms
    per launch of the median replay and the (min, median, max) over the
    replays."""
    sp = stream.cuda_stream
    with torch.cuda.stream(stream):
        for i in range(warmup):
            launch_one(i, sp)
        torch.cuda.synchronize()
        hipgraph.begin_capture(sp)
        for i in range(steps):
            launch_one(warmup + i, sp)
        graph, exe = hipgraph.end_capture(sp)
        # one untimed replay so the graph's first-launch costs stay outside
        hipgraph.launch(exe, sp)
        torch.cuda.synchronize()
        times = []
        for _ in range(replays):
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            if before_replay is not None:
                before_replay(sp)
            torch.cuda.synchronize()
            e0.record(stream)
            hipgraph.launch(exe, sp)
            e1.record(stream)
            torch.cuda.synchronize()
            times.append(e0.elapsed_time(e1) / steps)
    hipgraph.destroy(graph, exe)
    times.sort()
    return times[len(times) // 2], (times[0], times[len(times) // 2], times[-1])


def cold_buffers(L):
    """KV buffers a decode at L rotates to be HBM-cold: more than 320 MB
    together (the MALL holds 256 MB), and at least 8 (C3: 8 x 67 MB)."""
    return max(8, -(-320_000_000 // decode_bytes(L)))


_flush_buf = None


def flush_mall(torch, sp):
    """Reads 512 MB of unrelated device memory on stream `sp`, so that no
    K/V byte of an earlier replay is still in the MALL (256 MB)."""
    global _flush_buf
    if _flush_buf is None:
        _flush_buf = torch.ones(128 << 20, dtype=torch.int32, device="cuda")
    n = _flush_buf.numel() * 4 // 2
    p = _flush_buf.data_ptr()
    sink = torch.zeros(4, dtype=torch.int32, device="cuda")
    assert bench_lib().attn_bench_read2(p, n, p + n, n, sink.data_ptr(), 1024, sp) == 0


def bench_decode(torch, A, hipgraph, L, nbuf, steps, warmup, seed=3, flush=False, replays=7):
    """Flash-Decode over `nbuf` distinct KV buffers in rotation (with `flush`,
    the MALL is flushed before every timed replay)."""
    dev = torch.device("cuda:0")
    q = rand16(torch, Q_DIM, seed)
    ks = [rand16(torch, (L + 1) * KV_DIM, seed + 1 + 2 * b) for b in range(nbuf)]
    vs = [rand16(torch, (L + 1) * KV_DIM, seed + 2 + 2 * b) for b in range(nbuf)]
    po, pm, ps = A.decode_workspace(HQ, L, D, device=dev)
    out = torch.empty(Q_DIM, dtype=torch.float16, device=dev)
    lib = A.lib()
    args = [(q.data_ptr(), ks[b].data_ptr(), vs[b].data_ptr(), out.data_ptr(), po.data_ptr(),
             pm.data_ptr(), ps.data_ptr()) for b in range(nbuf)]

    def launch(i, sp):
        a = args[i % nbuf]
        rc = lib.attn_decode(*a, 1, L, L - 1, HQ, HKV, D, QKV, KV_DIM, sp, None, None)
        assert rc == 0

    stream = torch.cuda.Stream()
    ms, spread = time_graph(torch, A, hipgraph, launch, steps, warmup, stream, replays=replays,
                            before_replay=(lambda sp: flush_mall(torch, sp)) if flush else None)
    del ks, vs
    return ms, spread


def device_warmup(torch, seconds=0.25):
    """Streams a 256 MB buffer through torch elementwise kernels (distinct
    from every kernel a profile of this run reports) for `seconds` before
    anything is timed, so that the first timed replays do not meet the GPU's
    idle clock and power state."""
    buf = torch.ones(64 << 20, dtype=torch.float32, device="cuda")
    t0 = time.time()
    while time.time() - t0 < seconds:
        for _ in range(20):
            buf.mul_(1.0)
        torch.cuda.synchronize()
    del buf


_bench_lib = None


def bench_lib():
    """libattn_bench.so: measurement helpers (streaming-read ceiling, the
    reference engine's per-token decode loop); not part of the attention
    library."""
    global _bench_lib
    if _bench_lib is not None:
        return _bench_lib
    import ctypes
    lib = ctypes.CDLL(str(ROOT / "llm-inference_amd" / "lib" / "libattn_bench.so"))
    vp, sz = ctypes.c_void_p, ctypes.c_size_t
    lib.attn_bench_read2.argtypes = [vp, sz, vp, sz, vp, ctypes.c_uint, vp]
    lib.attn_bench_read2.restype = ctypes.c_int
    lib.attn_bench_engine_decode.argtypes = [vp] * 8 + [sz] * 7 + [ctypes.c_int, vp]
    lib.attn_bench_engine_decode.restype = ctypes.c_int
    lib.attn_bench_empty.argtypes = [vp, ctypes.c_uint, ctypes.c_uint, vp]
    lib.attn_bench_empty.restype = ctypes.c_int
    _bench_lib = lib
    return lib


def bench_launch_floor(torch, A, hipgraph, kernels, wgs, steps, warmup):
    """ms per step of `kernels` dependent launches of an empty kernel (`wgs`
    workgroups of 256 threads), timed like the short prompts: the fixed cost
    a one- or two-kernel call pays in a graph before any work."""
    sink = torch.zeros(wgs, dtype=torch.int32, device="cuda")
    blib = bench_lib()

    def launch(i, sp):
        for _ in range(kernels):
            assert blib.attn_bench_empty(sink.data_ptr(), wgs, 0, sp) == 0

    return time_graph(torch, A, hipgraph, launch, steps, warmup, torch.cuda.Stream())[0]


def bench_read_ceiling(torch, A, hipgraph, L, nbuf, steps, warmup, wgs=1024, seed=3,
                       flush=False):
    """A plain streaming read of the same bytes a decode call reads (K and V
    rows 0..L-1 of one of `nbuf` rotated buffers), timed exactly as
    bench_decode times the decode: the ceiling for a decode call."""
    ks = [rand16(torch, (L + 1) * KV_DIM, seed + 1 + 2 * b) for b in range(nbuf)]
    vs = [rand16(torch, (L + 1) * KV_DIM, seed + 2 + 2 * b) for b in range(nbuf)]
    sink = torch.zeros(4, dtype=torch.int32, device="cuda")
    blib = bench_lib()

    def launch(i, sp):
        b = i % nbuf
        assert blib.attn_bench_read2(ks[b].data_ptr(), L * KV_DIM * 2, vs[b].data_ptr(),
                                     L * KV_DIM * 2, sink.data_ptr(), wgs, sp) == 0

    ms, spread = time_graph(torch, A, hipgraph, launch, steps, warmup, torch.cuda.Stream(),
                            before_replay=(lambda sp: flush_mall(torch, sp)) if flush else None)
    del ks, vs
    return ms, spread


def bench_engine_c5(torch, A, layers=36, first_pos=32768, tokens=24, fused=False):
    """The reference engine's decode loop over the attention path
    (model_inference.hpp:76-134, in C++ through the reference launch API):
    the first token captured in global mode, then per token every layer's
    nodes patched (3 updaters per layer, or 1 for the fused RoPE + decode),
    hipGraphLaunch and a stream synchronize.  Positions first_pos ..
    first_pos + tokens - 1, so kv_len runs from 32769 (C5) upward."""
    import ctypes
    dev = torch.device("cuda:0")
    S = first_pos + tokens
    cache = torch.empty(layers * 2 * S * KV_DIM, dtype=torch.float16, device=dev)
    g = torch.Generator(device=dev)
    for l in range(layers):
        g.manual_seed(500 + l)
        o = l * 2 * S * KV_DIM
        cache[o:o + 2 * S * KV_DIM].normal_(generator=g)
    qkv = rand16(torch, layers * QKV, 499)
    cos, sin = A.rope_tables(S, D, THETA)
    dcos, dsin = cos.to(dev), sin.to(dev)
    po, pm, ps = A.decode_workspace(HQ, S, D, device=dev)
    out = torch.empty(layers * Q_DIM, dtype=torch.float16, device=dev)
    res = (ctypes.c_double * 6)()
    rc = bench_lib().attn_bench_engine_decode(
        cache.data_ptr(), qkv.data_ptr(), dcos.data_ptr(), dsin.data_ptr(), out.data_ptr(),
        po.data_ptr(), pm.data_ptr(), ps.data_ptr(), layers, HQ, HKV, D, S, first_pos, tokens,
        1 if fused else 0, res)
    assert rc == 0, rc
    del cache
    return {"host_patch_us": res[0], "per_token_us": res[1], "gpu_us": res[2],
            "capture_ms": res[3], "per_token_min_us": res[4], "per_token_max_us": res[5],
            "tokens": tokens - 1, "kv_len": f"{first_pos + 2}..{first_pos + tokens}",
            "nodes": layers * (1 if fused else 3)}


def bench_qkv(torch, A, hipgraph, mode, nbuf, steps, warmup, pos=4000, seed=8):
    """One decode step's QKV projection over `nbuf` distinct weight matrices
    in rotation (24 x 12.6 MB exceeds the 256 MB last-level cache, as 36
    layers' weights do): mode "gemv" (launch_qkv_decode), "fused" (GEMV + RoPE
    + KV append in one kernel) or "two" (launch_qkv_decode then
    launch_rope_and_store_kv)."""
    dev = torch.device("cuda:0")
    ws = [rand16(torch, QKV * HIDDEN, seed + b, 1.0 / 45) for b in range(nbuf)]
    x = rand16(torch, HIDDEN, seed - 1)
    y = torch.empty(QKV, dtype=torch.float16, device=dev)
    cos, sin = A.rope_tables(pos + 1, D, THETA)
    dcos, dsin = cos.to(dev), sin.to(dev)
    cache = torch.empty(2 * (pos + 1) * KV_DIM, dtype=torch.float16, device=dev)
    kc, vc = cache.data_ptr(), cache.data_ptr() + 2 * (pos + 1) * KV_DIM
    yp, xp, cp, sp_ = y.data_ptr(), x.data_ptr(), dcos.data_ptr(), dsin.data_ptr()
    lib = A.lib()

    def launch(i, sp):
        w = ws[i % nbuf].data_ptr()
        if mode == "fused":
            rc = lib.attn_qkv_rope_store_kv_decode(xp, yp, w, kc, vc, cp, sp_, HIDDEN, HQ, HKV, D,
                                                   pos, 1, sp)
        else:
            rc = lib.attn_qkv_decode(xp, yp, w, HIDDEN, QKV, sp)
            if rc == 0 and mode == "two":
                rc = lib.attn_rope_store_kv(yp, yp + 2 * Q_DIM, yp + 2 * (Q_DIM + KV_DIM), kc,
                                            vc, cp, sp_, 1, HQ, HKV, D, QKV, QKV, pos, 1, sp)
        assert rc == 0

    ms, _ = time_graph(torch, A, hipgraph, launch, steps, warmup, torch.cuda.Stream())
    del ws
    return ms


def bench_qkv_prefill(torch, A, hipgraph, M, mode, steps, warmup, seed=9):
    """Prefill QKV projection of M tokens (2048 -> 3072), ms per call (graph of
    `steps` launches, median of 7 replays): mode "gemm" (launch_qkv_gemm),
    "fused" (GEMM + RoPE + KV append in one kernel) or "two"
    (launch_qkv_gemm then launch_rope_and_store_kv)."""
    dev = torch.device("cuda:0")
    x = rand16(torch, M * HIDDEN, seed)
    w = rand16(torch, QKV * HIDDEN, seed + 1, 1.0 / 45)
    y = torch.empty(M * QKV, dtype=torch.float16, device=dev)
    cos, sin = A.rope_tables(M, D, THETA)
    dcos, dsin = cos.to(dev), sin.to(dev)
    cache = torch.empty(2 * M * KV_DIM, dtype=torch.float16, device=dev)
    kc, vc = cache.data_ptr(), cache.data_ptr() + 2 * M * KV_DIM
    xp, yp, wp, cp, snp = x.data_ptr(), y.data_ptr(), w.data_ptr(), dcos.data_ptr(), dsin.data_ptr()
    lib = A.lib()

    def launch(i, sp):
        if mode == "fused":
            rc = lib.attn_qkv_gemm_rope_store_kv(xp, yp, wp, kc, vc, cp, snp, M, HIDDEN, HQ, HKV,
                                                 D, 0, 1, sp)
        else:
            rc = lib.attn_qkv_gemm(xp, yp, wp, M, HIDDEN, QKV, sp)
            if rc == 0 and mode == "two":
                rc = lib.attn_rope_store_kv(yp, yp + 2 * Q_DIM, yp + 2 * (Q_DIM + KV_DIM), kc, vc,
                                            cp, snp, M, HQ, HKV, D, QKV, QKV, 0, 1, sp)
        assert rc == 0

    return time_graph(torch, A, hipgraph, launch, steps, warmup, torch.cuda.Stream())[0]


def bench_prefill(torch, A, N, launches, warmup, seed=4, sigma=0.5):
    """Prefill ms per call: `warmup` untimed calls (the clock ramps for tens of
    calls under MFMA load), then `launches` calls each bracketed by its own
    HIP events on the launch stream.  Returns the median and (min, median,
    max)."""
    dev = torch.device("cuda:0")
    qkv = rand16(torch, N * QKV, seed, sigma)
    kc = rand16(torch, N * KV_DIM, seed + 1, sigma)
    vc = rand16(torch, N * KV_DIM, seed + 2, sigma)
    out = torch.empty(N * Q_DIM, dtype=torch.float16, device=dev)
    stream = torch.cuda.current_stream()
    for _ in range(warmup):
        A.prefill(qkv, kc, vc, out, N, HQ, HKV, D, QKV, KV_DIM)
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(launches)]
    for e0, e1 in ev:
        e0.record(stream)
        A.prefill(qkv, kc, vc, out, N, HQ, HKV, D, QKV, KV_DIM)
        e1.record(stream)
    torch.cuda.synchronize()
    times = sorted(e0.elapsed_time(e1) for e0, e1 in ev)
    med = times[len(times) // 2]
    return med, (times[0], med, times[-1])


def bench_prefill_graph(torch, A, hipgraph, N, steps, warmup, seed=2, sigma=1.0):
    """Prefill ms per call for short prompts, timed like the decode: one graph
    of `steps` launches, median of 7 replays (per-launch events would add
    their own ~2 us to a ~10 us kernel)."""
    dev = torch.device("cuda:0")
    qkv = rand16(torch, N * QKV, seed, sigma)
    kc = rand16(torch, N * KV_DIM, seed + 1, sigma)
    vc = rand16(torch, N * KV_DIM, seed + 2, sigma)
    out = torch.empty(N * Q_DIM, dtype=torch.float16, device=dev)
    lib = A.lib()

    def launch(i, sp):
        assert lib.attn_prefill(qkv.data_ptr(), kc.data_ptr(), vc.data_ptr(), out.data_ptr(), N,
                                HQ, HKV, D, QKV, KV_DIM, sp) == 0

    return time_graph(torch, A, hipgraph, launch, steps, warmup, torch.cuda.Stream())[0]


def bench_rope(torch, A, hipgraph, N, nbuf, steps, warmup, rotate=True, seed=6):
    dev = torch.device("cuda:0")
    cos, sin = A.rope_tables(N + 1, D, THETA)
    dcos, dsin = cos.to(dev), sin.to(dev)
    srcs = [rand16(torch, N * QKV, seed + b) for b in range(nbuf)]
    caches = [torch.empty(2 * N * KV_DIM, dtype=torch.float16, device=dev) for _ in range(nbuf)]
    lib = A.lib()

    def launch(i, sp):
        s, c = srcs[i % nbuf].data_ptr(), caches[i % nbuf].data_ptr()
        rc = lib.attn_rope_store_kv(s, s + 2 * Q_DIM, s + 2 * (Q_DIM + KV_DIM), c,
                                    c + 2 * N * KV_DIM, dcos.data_ptr(), dsin.data_ptr(), N, HQ,
                                    HKV, D, QKV, QKV, 0, 1 if rotate else 0, sp)
        assert rc == 0

    stream = torch.cuda.Stream()
    return time_graph(torch, A, hipgraph, launch, steps, warmup, stream)[0]


def bench_c5(torch, A, hipgraph, replays, layers=36, L=32769, producer="rope"):
    """36-layer attention-only decode step: per layer RoPE(+append) of one new
    token at position L-1 (NoPE on every 4th layer, model_inference.hpp:358)
    and Flash-Decode (split + merge) over L keys, captured as one 108-node
    graph.  producer "rope_fused" issues each layer's RoPE/append and decode
    as the decode's two kernels (attn_rope_store_kv_decode, 72 nodes).
    producer "qkv_fused" / "qkv_two" start each layer from a hidden vector
    instead: the QKV GEMV (2048 -> 3072, per-layer weights) fused with the
    RoPE/append (108 nodes) or as the reference's two launches (144 nodes).
    producer "o_proj_two" / "o_proj_fused" end each layer with the attention
    output projection (per-layer W_o [2048][2048], beta = 1 into one residual
    vector): the reference's launch after the merge (144 nodes) or the merge
    fused into it (attn_decode_out_proj with decode_out_proj_fused = 1, 108
    nodes)."""
    dev = torch.device("cuda:0")
    S = L
    cache = torch.empty(layers * 2 * S * KV_DIM, dtype=torch.float16, device=dev)
    g = torch.Generator(device=dev)
    for l in range(layers):
        g.manual_seed(500 + l)
        o = l * 2 * S * KV_DIM
        cache[o:o + 2 * S * KV_DIM].normal_(generator=g)
    qkv = torch.randn(layers, QKV, device=dev).to(torch.float16)
    cos, sin = A.rope_tables(S, D, THETA)
    dcos, dsin = cos.to(dev), sin.to(dev)
    po, pm, ps = A.decode_workspace(HQ, L, D, device=dev)
    out = torch.empty(layers, Q_DIM, dtype=torch.float16, device=dev)
    lib = A.lib()
    cb = cache.data_ptr()
    stream = torch.cuda.Stream()
    sp = stream.cuda_stream
    start_pos = L - 1

    if producer.startswith("qkv"):
        ws = rand16(torch, layers * QKV * HIDDEN, 600, 1.0 / 45)
        x = rand16(torch, HIDDEN, 599)
    if producer.startswith("o_proj"):
        wo = rand16(torch, layers * HIDDEN * Q_DIM, 700, 1.0 / 45)
        y = rand16(torch, HIDDEN, 701)
        ows = A.decode_out_proj_workspace(HQ, HIDDEN, device=dev)

    def enqueue():
        for l in range(layers):
            s = qkv[l].data_ptr()
            kc = cb + 2 * (l * 2 * S * KV_DIM)
            vc = kc + 2 * S * KV_DIM
            apply = 1 if (l + 1) % 4 != 0 else 0
            if producer == "rope_fused":
                rc = lib.attn_rope_store_kv_decode(
                    s, s + 2 * Q_DIM, s + 2 * (Q_DIM + KV_DIM), kc, vc, dcos.data_ptr(),
                    dsin.data_ptr(), out[l].data_ptr(), po.data_ptr(), pm.data_ptr(),
                    ps.data_ptr(), L, start_pos, HQ, HKV, D, 0, apply, sp, None, None)
                assert rc == 0
                continue
            if producer == "qkv_fused":
                rc = lib.attn_qkv_rope_store_kv_decode(
                    x.data_ptr(), s, ws.data_ptr() + 2 * l * QKV * HIDDEN, kc, vc,
                    dcos.data_ptr(), dsin.data_ptr(), HIDDEN, HQ, HKV, D, start_pos, apply, sp)
            else:
                rc = 0
                if producer == "qkv_two":
                    rc = lib.attn_qkv_decode(x.data_ptr(), s, ws.data_ptr() + 2 * l * QKV * HIDDEN,
                                             HIDDEN, QKV, sp)
                if rc == 0:
                    rc = lib.attn_rope_store_kv(s, s + 2 * Q_DIM, s + 2 * (Q_DIM + KV_DIM), kc,
                                                vc, dcos.data_ptr(), dsin.data_ptr(), 1, HQ, HKV,
                                                D, QKV, QKV, start_pos, apply, sp)
            assert rc == 0
            if producer == "o_proj_fused":
                rc = lib.attn_decode_out_proj(
                    s, kc, vc, out[l].data_ptr(), po.data_ptr(), pm.data_ptr(), ps.data_ptr(), L,
                    HQ, HKV, D, KV_DIM, wo.data_ptr() + 2 * l * HIDDEN * Q_DIM, y.data_ptr(),
                    HIDDEN, 1.0, ows.data_ptr(), sp, None, None)
                assert rc == 0
                continue
            rc = lib.attn_decode(s, kc, vc, out[l].data_ptr(), po.data_ptr(), pm.data_ptr(),
                                 ps.data_ptr(), 1, L, start_pos, HQ, HKV, D, QKV, KV_DIM, sp,
                                 None, None)
            assert rc == 0
            if producer == "o_proj_two":
                rc = lib.attn_out_proj_decode(out[l].data_ptr(), y.data_ptr(),
                                              wo.data_ptr() + 2 * l * HIDDEN * Q_DIM, HIDDEN, HQ,
                                              D, 1.0, sp)
                assert rc == 0

    with torch.cuda.stream(stream):
        if producer == "o_proj_fused":
            A.set_option("decode_out_proj_fused", 1)
        try:
            hipgraph.begin_capture(sp)
            enqueue()
            graph, exe = hipgraph.end_capture(sp)
        finally:
            A.set_option("decode_out_proj_fused", 0)
        hipgraph.launch(exe, sp)
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(replays):
            hipgraph.launch(exe, sp)
        e1.record(stream)
        torch.cuda.synchronize()
    hipgraph.destroy(graph, exe)
    ms = e0.elapsed_time(e1) / replays
    nrot = sum(1 for l in range(layers) if (l + 1) % 4 != 0)
    byts = layers * decode_bytes(L) + nrot * rope_bytes(1, True) + (layers - nrot) * rope_bytes(1, False)
    if producer.startswith("qkv"):
        byts += layers * qkv_bytes()
        del ws
    if producer.startswith("o_proj"):
        byts += layers * 2 * HIDDEN * Q_DIM
        del wo
    del cache
    return ms, byts


def cpu_baselines(torch, quick):
    """The reference's PyTorch CPU attention (python/reference.py:79-92)
    restated with the same torch calls (fp16 SDPA with repeat_interleave, all
    torch threads; kind "port", the reference file is not run) on a bounded
    sample of C3 decode calls (~10 s), plus prefill and RoPE samples, and the
    oracle (fp64 C, 1 thread) on a few decode calls."""
    import numpy as np
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle
    res = {}
    L = 32768
    rng = np.random.default_rng(3)
    q = rng.standard_normal(Q_DIM).astype(np.float16).view(np.uint16)
    k = rng.standard_normal(L * KV_DIM).astype(np.float16).view(np.uint16)
    v = rng.standard_normal(L * KV_DIM).astype(np.float16).view(np.uint16)
    # reference PyTorch CPU attention (python/reference.py:79-92), fp16
    import torch.nn.functional as F
    nthreads = torch.get_num_threads()
    qt = torch.from_numpy(q.view(np.float16)).view(1, HQ, 1, D)
    kt = torch.from_numpy(k.view(np.float16)).view(1, L, HKV, D).transpose(1, 2)
    vt = torch.from_numpy(v.view(np.float16)).view(1, L, HKV, D).transpose(1, 2)

    def dec():
        kk = kt.repeat_interleave(HQ // HKV, dim=1)
        vv = vt.repeat_interleave(HQ // HKV, dim=1)
        return F.scaled_dot_product_attention(qt, kk, vv)

    dec()
    budget = 2.0 if quick else 10.0
    times = []
    t_end = time.perf_counter() + budget
    while time.perf_counter() < t_end or len(times) < 5:
        t0 = time.perf_counter()
        dec()
        times.append(time.perf_counter() - t0)
    times.sort()
    dt = times[len(times) // 2]
    res["torch_decode"] = {"value": decode_bytes(L) / dt / 1e9, "unit": "GB/s",
                           "cores": nthreads, "kind": "port",
                           "sample": f"torch SDPA fp16 decode, C3 L=32768 (16 q / 4 kv heads, "
                                     f"D=128, K/V repeat_interleave), {len(times)} calls in "
                                     f"{sum(times):.1f} s, median {dt * 1e3:.2f} ms "
                                     f"(min {times[0] * 1e3:.2f}, max {times[-1] * 1e3:.2f})"}
    calls = 2 if quick else 8
    oracle.attention(q, k, v, 1, HQ, HKV, D, Q_DIM, KV_DIM, L, L - 1, causal=False)
    t0 = time.perf_counter()
    for _ in range(calls):
        oracle.attention(q, k, v, 1, HQ, HKV, D, Q_DIM, KV_DIM, L, L - 1, causal=False)
    dt = (time.perf_counter() - t0) / calls
    res["oracle"] = {"value": decode_bytes(L) / dt / 1e9, "unit": "GB/s", "cores": 1,
                     "kind": "port",
                     "sample": f"{calls} Flash-Decode calls at L=32768 (16 q / 4 kv heads, D=128) "
                               f"through the fp64 C oracle, {dt * 1e3:.1f} ms each"}
    # prefill sample: one GQA group (4 q heads, 1 kv head) at N = 8192 -> scaled
    N = 2048 if quick else 8192
    qp = torch.randn(1, 4, N, D).to(torch.float16)
    kp = torch.randn(1, 1, N, D).to(torch.float16).repeat_interleave(4, dim=1)
    vp = torch.randn(1, 1, N, D).to(torch.float16).repeat_interleave(4, dim=1)
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        F.scaled_dot_product_attention(qp, kp, vp, is_causal=True)
        times.append(time.perf_counter() - t0)
    dt = float(np.median(times))
    flops = 2 * 4 * D * N * (N + 1)
    res["torch_prefill"] = {"value": flops / dt / 1e12, "unit": "TFLOP/s", "cores": nthreads,
                            "kind": "port",
                            "sample": f"torch SDPA fp16 causal prefill, N={N}, 4 q heads of one "
                                      f"KV group (1/4 of C4), median of 3: {dt:.2f} s"}
    # RoPE as the reference's PyTorch path applies it (python/reference.py:63-73:
    # fp16 cos/sin, q * cos + rotate_half(q) * sin) on C4's 8192 tokens
    Nr = 8192
    pos = torch.arange(Nr, dtype=torch.float32)
    inv = 1.0 / (THETA ** (torch.arange(0, D, 2, dtype=torch.float32) / D))
    ang = torch.outer(pos, inv)
    cos = torch.cat([ang.cos(), ang.cos()], dim=-1).to(torch.float16)[:, None, :]
    sin = torch.cat([ang.sin(), ang.sin()], dim=-1).to(torch.float16)[:, None, :]
    qr = torch.randn(Nr, HQ, D).to(torch.float16)
    kr = torch.randn(Nr, HKV, D).to(torch.float16)

    def rot(x):
        x1, x2 = x[..., :D // 2], x[..., D // 2:]
        return x * cos + torch.cat([-x2, x1], dim=-1) * sin

    rot(qr), rot(kr)
    times = []
    for _ in range(5):
        t0 = time.perf_counter()
        rot(qr), rot(kr)
        times.append(time.perf_counter() - t0)
    dt = float(np.median(times))
    res["torch_rope"] = {"value": rope_bytes(Nr) / dt / 1e9, "unit": "GB/s", "cores": nthreads,
                         "kind": "port",
                         "sample": f"torch fp16 rotate-half RoPE of Q and K, N={Nr} "
                                   f"(algorithmic bytes as the fused kernel), median of 5: "
                                   f"{dt * 1e3:.2f} ms"}
    res["host"] = {"cpu_count": os.cpu_count(), "torch_threads": nthreads,
                   "cpu": platform.processor() or platform.machine(),
                   "torch": torch.__version__}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    res["host"]["cpu"] = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return res


def profile_workload(torch, A):
    """Eager launches of every hot kernel at its headline shape, for hardware
    counter passes (one dispatch per kernel call, no graph)."""
    dev = torch.device("cuda:0")
    L, nbuf = 32768, 8
    q = rand16(torch, Q_DIM, 3)
    ks = [rand16(torch, (L + 1) * KV_DIM, 4 + 2 * b) for b in range(nbuf)]
    vs = [rand16(torch, (L + 1) * KV_DIM, 5 + 2 * b) for b in range(nbuf)]
    po, pm, ps = A.decode_workspace(HQ, L, D, device=dev)
    out = torch.empty(Q_DIM, dtype=torch.float16, device=dev)
    for i in range(16):
        A.decode(q, ks[i % nbuf], vs[i % nbuf], out, po, pm, ps, 1, L, L - 1, HQ, HKV, D, QKV,
                 KV_DIM)
    torch.cuda.synchronize()
    log(f"profile: 16 decode calls L={L} (algorithmic {decode_bytes(L)} B each)")
    rcos, rsin = A.rope_tables(L, D, THETA)
    rcos, rsin = rcos.to(dev), rsin.to(dev)
    knew, vnew = rand16(torch, KV_DIM, 30), rand16(torch, KV_DIM, 31)
    for i in range(16):
        A.rope_store_kv_decode(q, knew, vnew, ks[i % nbuf], vs[i % nbuf], rcos, rsin, out, po, pm,
                               ps, L, L - 1, HQ, HKV, D, True)
    torch.cuda.synchronize()
    log(f"profile: 16 fused RoPE + append + decode calls L={L}")
    del ks, vs
    N = 8192
    qkv = rand16(torch, N * QKV, 4, 0.5)
    kc = rand16(torch, N * KV_DIM, 5, 0.5)
    vc = rand16(torch, N * KV_DIM, 6, 0.5)
    o = torch.empty(N * Q_DIM, dtype=torch.float16, device=dev)
    for _ in range(3):
        A.prefill(qkv, kc, vc, o, N, HQ, HKV, D, QKV, KV_DIM)
    torch.cuda.synchronize()
    log(f"profile: 3 prefill calls N={N}")
    cos, sin = A.rope_tables(N, D, THETA)
    dcos, dsin = cos.to(dev), sin.to(dev)
    cache = torch.empty(2 * N * KV_DIM, dtype=torch.float16, device=dev)
    lib = A.lib()
    s, c = qkv.data_ptr(), cache.data_ptr()
    for _ in range(3):
        rc = lib.attn_rope_store_kv(s, s + 2 * Q_DIM, s + 2 * (Q_DIM + KV_DIM), c,
                                    c + 2 * N * KV_DIM, dcos.data_ptr(), dsin.data_ptr(), N, HQ,
                                    HKV, D, QKV, QKV, 0, 1, torch.cuda.current_stream().cuda_stream)
        assert rc == 0
    torch.cuda.synchronize()
    log(f"profile: 3 rope+append calls N={N} (algorithmic {rope_bytes(N)} B each)")
    del qkv, kc, vc, o, cache
    ws = [rand16(torch, QKV * HIDDEN, 40 + b, 1.0 / 45) for b in range(24)]
    x = rand16(torch, HIDDEN, 39)
    y = torch.empty(QKV, dtype=torch.float16, device=dev)
    kc1 = torch.empty(2 * N * KV_DIM, dtype=torch.float16, device=dev)
    sp = torch.cuda.current_stream().cuda_stream
    for i in range(24):
        assert lib.attn_qkv_decode(x.data_ptr(), y.data_ptr(), ws[i].data_ptr(), HIDDEN, QKV,
                                   sp) == 0
    for i in range(24):
        assert lib.attn_qkv_rope_store_kv_decode(
            x.data_ptr(), y.data_ptr(), ws[i].data_ptr(), kc1.data_ptr(),
            kc1.data_ptr() + 2 * N * KV_DIM, dcos.data_ptr(), dsin.data_ptr(), HIDDEN, HQ, HKV,
            D, N - 1, 1, sp) == 0
    torch.cuda.synchronize()
    log(f"profile: 24 + 24 decode QKV calls (GEMV, fused), weights cold "
        f"(algorithmic {qkv_bytes()} B each)")
    del ws
    xp = rand16(torch, N * HIDDEN, 38)
    wp = rand16(torch, QKV * HIDDEN, 37, 1.0 / 45)
    yq = torch.empty(N * QKV, dtype=torch.float16, device=dev)
    for _ in range(3):
        A.qkv_gemm(xp, yq, wp, N, HIDDEN, QKV)
    for _ in range(3):
        A.qkv_gemm_rope_store_kv(xp, yq, wp, kc1, kc1.data_ptr() + 2 * N * KV_DIM, dcos, dsin, N,
                                 HIDDEN, HQ, HKV, D, 0, True)
    torch.cuda.synchronize()
    log(f"profile: 3 + 3 prefill QKV calls N={N} (GEMM, fused; {2 * N * QKV * HIDDEN} FLOP each)")
    del xp, wp, yq
    src = torch.empty(128 << 20, dtype=torch.float16, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    log("profile: 3 device copies of 256 MiB (reads 268435456 B, writes 268435456 B each)")


def decode_timeline(torch, A, hipgraph, steps=20, warmup=5):
    """Per-segment timeline of decode calls from the instrumented library
    (libattn_timeline.so: the product's sources compiled with
    ATTN_DECODE_TIMELINE, whose split and merge kernels store s_memrealtime
    stamps, 100 MHz, at fixed points of every workgroup).  Each length runs
    as bench_decode runs it (graph of `steps` calls, cold over 8 rotated KV
    buffers from 4096 keys); the records of the last replay's calls 2..steps
    are reduced per call relative to the call's first split workgroup entry,
    then the median over the calls is reported.  Also: the plain streaming
    read of the same bytes, cold and warm (one buffer, MALL-resident)."""
    import ctypes
    import numpy as np
    lib = A.lib()
    lib.attn_timeline_set.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    lib.attn_timeline_set.restype = ctypes.c_int
    lib.attn_timeline_slot_words.argtypes = []
    lib.attn_timeline_slot_words.restype = ctypes.c_size_t
    words = lib.attn_timeline_slot_words()
    split_words, merge_base = 16, 16 * 1024
    slots = warmup + steps + 1
    buf = torch.zeros(slots * words, dtype=torch.int64, device="cuda")
    tick_us = 0.01  # s_memrealtime: 100 MHz
    out = {"what": "instrumented build (libattn_timeline.so); us after the first split "
                   "workgroup's entry, median over the calls of the last replay",
           "lengths": {}}
    for L in (32768, 65536, 16384, 4096, 254):
        plan = A.decode_plan(L, HQ, HKV, D, KV_DIM)
        groups = HKV // {1: 4, 2: 2, 3: 1}[plan["path"]]
        nsplit_wg = groups * plan["nsplit"]
        whole = plan["nsplit"] == 1  # one kernel: no merge records
        nmerge = HQ * (D // 4)
        buf.zero_()
        torch.cuda.synchronize()
        assert lib.attn_timeline_set(buf.data_ptr(), slots) == 0
        ms, _ = bench_decode(torch, A, hipgraph, L, 8 if L >= 4096 else 1, steps, warmup)
        rec = buf.view(slots, words).cpu().numpy()
        calls = []
        for s in range(warmup + 1, warmup + steps):
            r = rec[s]
            sp = r[:split_words * nsplit_wg].reshape(nsplit_wg, split_words).astype(np.float64)
            mg = r[merge_base:merge_base + 4 * nmerge].reshape(nmerge, 4).astype(np.float64)
            t0 = sp[:, 0].min()
            rel = lambda x: (x - t0) * tick_us  # noqa: E731
            wc = sp[:, 2:10]
            wc_any = wc[wc > 0]
            wg_comp = wc.max(axis=1)           # each workgroup's last wave computed
            last_wg = int(np.argmax(sp[:, 11]))  # the workgroup whose stores were acked last
            c = {
                "split_entry_last": rel(sp[:, 0].max()),
                "loads_issued_median": rel(np.median(sp[:, 1])),
                "loads_issued_last": rel(sp[:, 1].max()),
                "wave_computed_first": rel(wc_any.min()),
                "wave_computed_median": rel(np.median(wc_any)),
                "wave_computed_last": rel(wc_any.max()),
                "barrier_passed_last": rel(sp[:, 14].max()),
                "fold_done_last": rel(sp[:, 10].max()),
                "stores_acked_last": rel(sp[:, 11].max()),
                "wg_barrier_after_last_wave_median": float(np.median(sp[:, 14] - wg_comp)) * tick_us,
                "wg_fold_after_barrier_median": float(np.median(sp[:, 10] - sp[:, 14])) * tick_us,
                "wg_acked_after_fold_median": float(np.median(sp[:, 11] - sp[:, 10])) * tick_us,
                "last_wg_computed": rel(wg_comp[last_wg]),
                "last_wg_barrier": rel(sp[last_wg, 14]),
                "last_wg_fold": rel(sp[last_wg, 10]),
            }
            if not whole:
                c.update({
                    "merge_entry_first": rel(mg[:, 0].min()),
                    "merge_entry_last": rel(mg[:, 0].max()),
                    "merge_states_folded_median": rel(np.median(mg[:, 1])),
                    "merge_states_folded_last": rel(mg[:, 1].max()),
                    "merge_stored_last": rel(mg[:, 2].max()),
                })
            if s + 1 < warmup + steps:
                nxt = rec[s + 1][:split_words * nsplit_wg].reshape(nsplit_wg, split_words)
                c["next_call_split_entry"] = rel(float(nxt[:, 0].min()))
            xcc = sp[:, 13].astype(int)
            c["wave_computed_last_per_xcd"] = {int(x): rel(wg_comp[xcc == x].max())
                                               for x in np.unique(xcc)}
            # per wave slot of the workgroup (waves w and w + 4 share a SIMD)
            c["wave_computed_median_per_slot"] = {
                w: rel(float(np.median(wc[wc[:, w] > 0, w]))) for w in range(8)
                if (wc[:, w] > 0).any()}
            calls.append(c)
        med = {}
        for k in calls[0]:
            if k in ("wave_computed_last_per_xcd", "wave_computed_median_per_slot"):
                med[k] = {x: float(np.median([cc[k][x] for cc in calls if x in cc[k]]))
                          for x in calls[0][k]}
            else:
                vals = [cc[k] for cc in calls if k in cc]
                med[k] = float(np.median(vals))
        xcc0 = rec[warmup + 1][:split_words * nsplit_wg].reshape(nsplit_wg, split_words)[:, 13]
        med["split_workgroups_per_xcd"] = {int(x): int((xcc0 == x).sum()) for x in np.unique(xcc0)}
        med["us_per_call_instrumented"] = ms * 1e3
        med["plan"] = plan
        out["lengths"][str(L)] = med
        log(f"timeline L={L}: {ms * 1e3:.2f} us per call (instrumented); "
            + ", ".join(f"{k} {v:.2f}" for k, v in med.items() if isinstance(v, float)))
    for L in (32768, 65536, 4096):
        cold, _ = bench_read_ceiling(torch, A, hipgraph, L, 8, steps, warmup)
        warm, _ = bench_read_ceiling(torch, A, hipgraph, L, 1, steps, warmup)
        out.setdefault("read_ceiling", {})[str(L)] = {"cold_us": cold * 1e3, "warm_us": warm * 1e3}
        log(f"read ceiling L={L}: cold {cold * 1e3:.2f} us, warm {warm * 1e3:.2f} us")
    for wgs in (256, 512, 2048):
        cold, _ = bench_read_ceiling(torch, A, hipgraph, 32768, 8, steps, warmup, wgs=wgs)
        out["read_ceiling"]["32768"][f"cold_us_{wgs}_workgroups"] = cold * 1e3
        log(f"read ceiling L=32768, {wgs} workgroups: cold {cold * 1e3:.2f} us")
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--quick", action="store_true", help="headline only, short CPU sample")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    ap.add_argument("--profile", action="store_true",
                    help="eager launches only, for rocprofv3 --pmc passes: 16 cold C3 decode "
                         "calls, 3 C4 prefills, 3 RoPE+append at 8192 tokens, 24 + 24 decode "
                         "QKV projections (GEMV, fused), 3 + 3 prefill QKV projections at 8192 "
                         "tokens (GEMM, fused) and a 256 MiB device copy that calibrates the "
                         "byte counters")
    ap.add_argument("--timeline", action="store_true",
                    help="per-segment timeline of decode calls from the instrumented library "
                         "(libattn_timeline.so), plus the streaming read cold and warm")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only: the attention hot path runs "
                                   "on one device (it would shard over KV heads or context, not "
                                   "built here); run with --gpus 1"}))
        sys.exit(2)

    import torch
    import attn_mi355x as A
    from attn_mi355x import hipgraph
    if args.timeline:
        A.LIB_PATH = A.PKG_ROOT / "lib" / "libattn_timeline.so"
    A.lib()
    props = torch.cuda.get_device_properties(0)
    log(f"device {props.name} {props.gcnArchName} CUs={props.multi_processor_count}")
    steps, warmup = args.steps, args.warmup
    if args.profile:
        profile_workload(torch, A)
        return
    if args.timeline:
        print(json.dumps({"timeline": decode_timeline(torch, A, hipgraph)}), flush=True)
        return

    # ---- headline: C3 decode at L=32768, cold (8 rotated KV buffers); the
    # median of 15 replays of `steps` calls, after a device warm-up
    device_warmup(torch)
    L = 32768
    plan = A.decode_plan(L, HQ, HKV, D, KV_DIM)
    ms, spread = bench_decode(torch, A, hipgraph, L, 8, steps, warmup, replays=15)
    gbs = decode_bytes(L) / (ms * 1e-3) / 1e9
    log(f"decode L={L} cold: {ms * 1e3:.2f} us  {gbs:.0f} GB/s  ({100 * gbs / PEAK_HBM_GBS:.1f}% of peak)"
        f" [replays min/median/max {spread[0] * 1e3:.2f}/{spread[1] * 1e3:.2f}/"
        f"{spread[2] * 1e3:.2f} us] plan={plan}")
    detail = {"decode": {}}
    detail["decode"][str(L)] = {"cold_us": ms * 1e3, "cold_GBps": gbs, "plan": plan,
                                "cold_replays_us": [t * 1e3 for t in spread],
                                "replays": 15, "steps_per_replay": steps}
    # the same rotated K/V bytes through a plain streaming read, timed the same way
    rms, rspread = bench_read_ceiling(torch, A, hipgraph, L, 8, steps, warmup)
    rgbs = decode_bytes(L) / (rms * 1e-3) / 1e9
    detail["read_ceiling"] = {str(L): {"us": rms * 1e3, "GBps": rgbs,
                                       "replays_us": [t * 1e3 for t in rspread]},
                              "what": "streaming read of the same K/V rows of 8 rotated "
                                      "buffers (1024 workgroups x 512 threads, 16-byte "
                                      "non-temporal loads), graph of K calls, median of 7"}
    log(f"read ceiling L={L}: {rms * 1e3:.2f} us {rgbs:.0f} GB/s; decode at "
        f"{100 * rms / ms:.1f}% of it")

    # ---- C4 prefill at 8192 tokens
    N = 8192
    pms, pspread = bench_prefill(torch, A, N, 60, 40)
    tflops = prefill_flops(N) / (pms * 1e-3) / 1e12
    log(f"prefill N={N}: {pms * 1e3:.1f} us  {tflops:.1f} TFLOP/s ({100 * tflops / PEAK_FP16_TFLOPS:.1f}% of fp16 peak)"
        f" [launches min/median/max {pspread[0] * 1e3:.1f}/{pspread[1] * 1e3:.1f}/"
        f"{pspread[2] * 1e3:.1f} us]")
    detail["prefill"] = {"8192": {"us": pms * 1e3, "TFLOPs": tflops,
                                  "launches_us": [t * 1e3 for t in pspread], "launches": 60}}

    if not args.quick:
        # cold from 4096 keys: K/V rotated over more than the MALL holds and
        # the MALL flushed before each replay; below, the 0.5 MB of C1 stays
        # in L2/MALL either way (cold = warm)
        for Lx in (254, 4096, 16384, 32768, 65536):
            if Lx >= 4096:
                cold, _ = bench_decode(torch, A, hipgraph, Lx, cold_buffers(Lx), steps, warmup,
                                       flush=True)
            warm, _ = bench_decode(torch, A, hipgraph, Lx, 1, steps, warmup)
            if Lx < 4096:
                cold = warm
            ent = detail["decode"].setdefault(str(Lx), {})
            if Lx == L:
                # the headline's own cold figure (8 rotated buffers, no flush)
                # stays cold_us; this flushed run is reported beside it
                ent.update({"cold_flushed_us": cold * 1e3,
                            "cold_flushed_GBps": decode_bytes(Lx) / cold / 1e6})
            else:
                ent.update({"cold_us": cold * 1e3, "cold_GBps": decode_bytes(Lx) / cold / 1e6})
            ent.update({"warm_us": warm * 1e3, "warm_GBps": decode_bytes(Lx) / warm / 1e6,
                        "plan": A.decode_plan(Lx, HQ, HKV, D, KV_DIM)})
            log(f"decode L={Lx}: cold {cold * 1e3:.2f} us ({decode_bytes(Lx) / cold / 1e6:.0f} GB/s)"
                f" warm {warm * 1e3:.2f} us ({decode_bytes(Lx) / warm / 1e6:.0f} GB/s)")
        for Lx in (4096, 65536):
            r, _ = bench_read_ceiling(torch, A, hipgraph, Lx, cold_buffers(Lx), steps, warmup,
                                      flush=True)
            detail["read_ceiling"][str(Lx)] = {"us": r * 1e3, "GBps": decode_bytes(Lx) / r / 1e6}
            log(f"read ceiling L={Lx}: {r * 1e3:.2f} us")
        p254 = bench_prefill_graph(torch, A, hipgraph, 254, steps, warmup)
        detail["prefill"]["254"] = {"us": p254 * 1e3, "TFLOPs": prefill_flops(254) / p254 / 1e9}
        log(f"prefill N=254: {p254 * 1e3:.1f} us")
        # mid-length prompts (each length's automatic form), median of 60
        # per-launch event timings after 20 warm-up launches
        for Nx in (1024, 2048, 4096):
            pm, (plo, _, phi) = bench_prefill(torch, A, Nx, 60, 20)
            detail["prefill"][str(Nx)] = {"us": pm * 1e3, "TFLOPs": prefill_flops(Nx) / pm / 1e9,
                                          "launches_us": [plo * 1e3, pm * 1e3, phi * 1e3]}
            log(f"prefill N={Nx}: {pm * 1e3:.1f} us ({prefill_flops(Nx) / pm / 1e9:.0f} TFLOP/s)")
        f1 = bench_launch_floor(torch, A, hipgraph, 1, 128, steps, warmup)
        f2 = bench_launch_floor(torch, A, hipgraph, 2, 128, steps, warmup)
        detail["launch_floor"] = {"one_kernel_us": f1 * 1e3, "two_kernels_us": f2 * 1e3,
                                  "workgroups": 128}
        log(f"launch floor (empty kernel, 128 workgroups, in a graph): one {f1 * 1e3:.2f} us, "
            f"two dependent {f2 * 1e3:.2f} us")
        r8k = bench_rope(torch, A, hipgraph, 8192, 4, max(20, steps // 4), 5)
        r254 = bench_rope(torch, A, hipgraph, 254, 1, steps, warmup)
        r1 = bench_rope(torch, A, hipgraph, 1, 1, steps, warmup)
        detail["rope_append"] = {
            "8192": {"us": r8k * 1e3, "GBps": rope_bytes(8192) / r8k / 1e6},
            "254": {"us": r254 * 1e3, "GBps": rope_bytes(254) / r254 / 1e6},
            "1": {"us": r1 * 1e3}}
        log(f"rope+append N=8192: {r8k * 1e3:.2f} us ({rope_bytes(8192) / r8k / 1e6:.0f} GB/s); "
            f"N=254 {r254 * 1e3:.2f} us; N=1 {r1 * 1e3:.2f} us")
        qk = {m: bench_qkv(torch, A, hipgraph, m, 24, steps, warmup)
              for m in ("gemv", "fused", "two")}
        detail["qkv_decode"] = {
            "gemv_us": qk["gemv"] * 1e3, "gemv_GBps": qkv_bytes() / qk["gemv"] / 1e6,
            "fused_us": qk["fused"] * 1e3, "two_kernel_us": qk["two"] * 1e3}
        log(f"QKV decode GEMV 2048->3072 cold: {qk['gemv'] * 1e3:.2f} us "
            f"({qkv_bytes() / qk['gemv'] / 1e6:.0f} GB/s); fused +RoPE+append "
            f"{qk['fused'] * 1e3:.2f} us vs two launches {qk['two'] * 1e3:.2f} us")
        qp = {}
        for Mq in (8192, 254):
            r = {m: bench_qkv_prefill(torch, A, hipgraph, Mq, m, 20, 20)
                 for m in ("gemm", "fused", "two")}
            fl = 2 * Mq * QKV * HIDDEN
            qp[str(Mq)] = {"gemm_us": r["gemm"] * 1e3, "gemm_TFLOPs": fl / r["gemm"] / 1e9,
                           "fused_us": r["fused"] * 1e3, "two_kernel_us": r["two"] * 1e3}
            log(f"QKV prefill GEMM {Mq}x2048->3072: {r['gemm'] * 1e3:.1f} us "
                f"({fl / r['gemm'] / 1e9:.0f} TFLOP/s); fused +RoPE+append {r['fused'] * 1e3:.1f} us "
                f"vs two launches {r['two'] * 1e3:.1f} us")
        detail["qkv_prefill"] = qp
        c5ms, c5b = bench_c5(torch, A, hipgraph, 10)
        detail["c5_36_layer_step"] = {"us": c5ms * 1e3, "bytes": c5b,
                                      "GBps": c5b / c5ms / 1e6,
                                      "pct_of_hbm_peak": 100 * c5b / c5ms / 1e6 / PEAK_HBM_GBS}
        log(f"C5 36-layer decode step: {c5ms * 1e3:.1f} us ({c5b / c5ms / 1e6:.0f} GB/s)")
        c5fms, c5fb = bench_c5(torch, A, hipgraph, 10, producer="rope_fused")
        detail["c5_36_layer_step_fused_rope_decode"] = {
            "us": c5fms * 1e3, "bytes": c5fb, "GBps": c5fb / c5fms / 1e6,
            "pct_of_hbm_peak": 100 * c5fb / c5fms / 1e6 / PEAK_HBM_GBS}
        log(f"C5 with RoPE/append fused into the decode kernels: {c5fms * 1e3:.1f} us "
            f"({c5fb / c5fms / 1e6:.0f} GB/s)")
        for fused in (False, True):
            eng = bench_engine_c5(torch, A, fused=fused)
            key = "c5_engine_loop_fused_rope_decode" if fused else "c5_engine_loop"
            eng["GBps"] = c5b / (eng["gpu_us"] * 1e-6) / 1e9
            detail[key] = eng
            log(f"C5 engine loop ({'fused RoPE + decode' if fused else 'RoPE node + decode'}): "
                f"{eng['per_token_us']:.1f} us per token, host patch {eng['host_patch_us']:.1f} us, "
                f"GPU {eng['gpu_us']:.1f} us")
        c5q = {p: bench_c5(torch, A, hipgraph, 10, producer=p) for p in ("qkv_fused", "qkv_two")}
        detail["c5_with_qkv_projection"] = {
            p: {"us": v[0] * 1e3, "bytes": v[1], "GBps": v[1] / v[0] / 1e6} for p, v in c5q.items()}
        log(f"C5 with the QKV projection: fused producer {c5q['qkv_fused'][0] * 1e3:.1f} us, "
            f"GEMV + RoPE {c5q['qkv_two'][0] * 1e3:.1f} us")
        c5o = {p: bench_c5(torch, A, hipgraph, 10, producer=p)
               for p in ("o_proj_two", "o_proj_fused")}
        detail["c5_with_out_projection"] = {
            p: {"us": v[0] * 1e3, "bytes": v[1], "GBps": v[1] / v[0] / 1e6} for p, v in c5o.items()}
        log(f"C5 with o_proj: split + merge + GEMV {c5o['o_proj_two'][0] * 1e3:.1f} us, "
            f"split + merge fused into o_proj {c5o['o_proj_fused'][0] * 1e3:.1f} us")

    cpu = None
    if not args.no_cpu:
        log("CPU baselines ...")
        cpu = cpu_baselines(torch, args.quick)
        detail["cpu"] = cpu
        log(f"CPU oracle decode {cpu['oracle']['value']:.2f} GB/s; torch CPU decode "
            f"{cpu['torch_decode']['value']:.2f} GB/s; torch CPU prefill "
            f"{cpu['torch_prefill']['value']:.3f} TFLOP/s; torch CPU RoPE "
            f"{cpu['torch_rope']['value']:.1f} GB/s")

    traffic = None
    tf = ROOT / "profiles" / "decode_traffic.json"
    if tf.exists():
        try:
            traffic = json.loads(tf.read_text()).get("hbm_bytes_per_launch")
        except (ValueError, OSError):
            traffic = None

    line = {
        "metric": "decode-attn HBM GB/s (% of peak) @32K ctx; prefill-attn TFLOPS @8K tokens",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic, seeded N(0,1) (prefill N(0,0.5))",
        "config": {"workload": "C3 Flash-Decode: 1 query token, 16 query heads / 4 KV heads, "
                               "head_dim 128, L=32768, KV rotated over 8 buffers (HBM-cold)",
                   "kv_len": L, "num_heads": HQ, "num_kv_heads": HKV, "head_dim": D,
                   "kv_buffers": 8, "parallelism": "single-gpu"},
        "decode_pct_of_hbm_peak": round(100 * gbs / PEAK_HBM_GBS, 2),
        "prefill": {"workload": "C4 causal GQA prefill, N=8192 tokens, 16/4 heads, D=128",
                    "us": round(pms * 1e3, 2), "tflops": round(tflops, 2),
                    "pct_of_fp16_peak": round(100 * tflops / PEAK_FP16_TFLOPS, 2)},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": traffic},
        "roofline_prefill": {"bound": "mfma", "achieved": round(tflops, 2),
                             "peak": PEAK_FP16_TFLOPS, "unit": "TFLOP/s",
                             "frac": round(tflops / PEAK_FP16_TFLOPS, 4), "traffic": None},
        "cpu_baseline": (cpu or {}).get("torch_decode"),
        "detail": detail,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
