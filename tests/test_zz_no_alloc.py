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
    for L, seed in ((32768, 71), (4096, 72)):
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
    group 16) at L = 65536 need 64 x 128 states of 520 bytes, more than
    ATTN_DECODE_NOALLOC_SCRATCH_BYTES (2 MiB).  The pointers are never
    dereferenced (the call returns before any launch)."""
    lib = attn.lib()
    p = attn.decode_plan(65536, 64, 4, 128)
    assert p["path"] != 0 and 64 * p["nstate"] * 520 > (2 << 20), p
    print(f"[case] noalloc rejection plan={p}", flush=True)
    assert lib.attn_decode_noalloc(256, 256, 256, 256, 65536, 64, 4, 128, 0, None) == 1
