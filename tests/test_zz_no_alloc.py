"""attn_decode_noalloc (no reference counterpart: attn_decode for callers that
cannot allocate) against attn_decode on the same inputs, through the C ABI:
two calls in a row on one GPU, the second with a smaller input (so a different
plan reuses the library's array), each bit-identical to attn_decode's output
(same plan and kernels) and within the north-star tolerance of the fp64
oracle."""
import numpy as np
import pytest
import torch

import oracle
from helpers import assert_close

pytestmark = pytest.mark.gpu

HQ, HKV, D = 16, 4, 128


def inputs(L, seed):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal(HQ * D).astype(np.float16)
    k = rng.standard_normal((L + 1) * HKV * D).astype(np.float16)
    v = rng.standard_normal((L + 1) * HKV * D).astype(np.float16)
    return q, k, v


def test_noalloc_decode_matches_workspace_decode(attn, gpu):
    lib = attn.lib()
    # the third call is a one-kernel plan (one split per KV head, no merge)
    for L, seed in ((32768, 71), (4096, 72), (254, 73)):
        plan = attn.decode_plan(L, HQ, HKV, D)
        print(f"[case] noalloc decode L={L} plan={plan}", flush=True)
        q, k, v = inputs(L, seed)
        dq, dk, dv = (torch.from_numpy(x).to(gpu) for x in (q, k, v))
        out_ref = torch.empty(HQ * D, dtype=torch.float16, device=gpu)
        out_na = torch.full((HQ * D,), float("nan"), dtype=torch.float16, device=gpu)
        po, pm, ps = attn.decode_workspace(HQ, L, D, device=gpu)
        attn.decode(dq, dk, dv, out_ref, po, pm, ps, 1, L, L - 1, HQ, HKV, D, 0, 0)
        rc = lib.attn_decode_noalloc(dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                                     out_na.data_ptr(), L, HQ, HKV, D, 0, None)
        assert rc == 0, rc
        torch.cuda.synchronize()
        a = out_na.cpu().numpy().view(np.uint16)
        b = out_ref.cpu().numpy().view(np.uint16)
        assert np.array_equal(a, b), L
        _, e = oracle.attention(q.view(np.uint16), k.view(np.uint16), v.view(np.uint16), 1, HQ,
                                HKV, D, HQ * D, HKV * D, L, L - 1, causal=False)
        assert_close(a, e.reshape(-1), 2e-3, 1e-2, f"noalloc L={L}")


def test_noalloc_rejects_plans_beyond_its_array(attn, gpu):
    """A plan needing more states than the array holds is rejected on the host
    before anything is enqueued: 64 query heads over 4 KV heads (the MFMA path,
    group 16) at L = 65536 need 64 x 128 states of 264 bytes (128 fp16 outputs, fp32 max and sum), more than
    ATTN_DECODE_NOALLOC_SCRATCH_BYTES (2 MiB).  The call is made inside a
    stream capture, so that even a regressed capacity check could only add
    kernel nodes to a graph that is never launched: the graph must come back
    empty, and the placeholder pointers are never dereferenced."""
    import ctypes
    from attn_mi355x import hipgraph
    lib = attn.lib()
    p = attn.decode_plan(65536, 64, 4, 128)
    assert p["path"] != 0 and 64 * p["nstate"] * 264 > (2 << 20), p
    print(f"[case] noalloc rejection plan={p}", flush=True)
    stream = torch.cuda.Stream()
    sp = stream.cuda_stream
    hip = hipgraph._hip
    hip.hipGraphGetNodes.argtypes = [ctypes.c_void_p, ctypes.c_void_p,
                                     ctypes.POINTER(ctypes.c_size_t)]
    hipgraph.begin_capture(sp)
    rc = lib.attn_decode_noalloc(256, 256, 256, 256, 65536, 64, 4, 128, 0, sp)
    graph = ctypes.c_void_p()
    hipgraph.check(hip.hipStreamEndCapture(sp, ctypes.byref(graph)), "hipStreamEndCapture")
    nodes = ctypes.c_size_t(0)
    try:
        hipgraph.check(hip.hipGraphGetNodes(graph, None, ctypes.byref(nodes)), "hipGraphGetNodes")
    finally:
        hip.hipGraphDestroy(graph)
    assert rc == 1, rc  # hipErrorInvalidValue
    assert nodes.value == 0


def test_noalloc_first_call_under_global_capture(gpu):
    """tests/cpp/test_noalloc_capture.cpp in a process of its own: the
    process's first attn_decode_noalloc call (which also looks up the array's
    address) made inside a hipStreamCaptureModeGlobal capture, then an eager
    call; whichever way the lookup goes under capture, the outputs equal
    attn_decode's bit for bit and a refused lookup is asked again."""
    import pathlib
    import subprocess
    exe = pathlib.Path(__file__).resolve().parent / "cpp" / "_build" / "test_noalloc_capture"
    assert exe.exists(), f"{exe} not built: run __graft_entry__.build()"
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    print(r.stdout)
    print(r.stderr)
    lines = [l for l in r.stdout.splitlines() if l.startswith(("PASS", "FAIL"))]
    assert len(lines) >= 4, r.stdout + r.stderr
    assert r.returncode == 0, r.stdout + r.stderr
