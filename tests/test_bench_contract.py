"""bench.py's measurement contract, checked on the CPU: the algorithmic work
each reported rate divides by, derived here from the tensors a call touches
(not from bench.py's formulas), and the refusal of a multi-GPU run."""
import json
import pathlib
import subprocess
import sys

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))
import bench  # noqa: E402  (no GPU work at import)

HQ, HKV, D = 16, 4, 128


def _nbytes(*shapes):
    return sum(np.zeros(s, dtype=np.float16).nbytes for s in shapes)


def test_decode_bytes_are_the_tensors_one_call_reads_and_writes():
    # q [Hq, D] read, K and V [L, Hkv, D] read once, out [Hq, D] written
    for L in (254, 4096, 16384, 32768, 65536):
        assert bench.decode_bytes(L) == _nbytes((HQ, D), (L, HKV, D), (L, HKV, D), (HQ, D)), L
    assert bench.decode_bytes(32768) == 67_117_056  # 8.39 us at 8 TB/s


def test_prefill_flops_count_every_causal_score_and_product():
    # each of Hq heads: query t scores keys 0..t (D multiply-adds) and
    # weights V over the same keys (D multiply-adds per output element)
    for N in (1, 2, 254, 8192):
        pairs = N * (N + 1) // 2
        assert bench.prefill_flops(N) == HQ * pairs * (2 * D + 2 * D), N
    assert bench.prefill_flops(8192) == 274_911_461_376


def test_rope_bytes_follow_the_fused_rows():
    # rotate: Q read + written, K read + cache row written, V read + cache
    # row written, cos and sin rows read; NoPE: K and V copied only
    N = 8192
    rotate = _nbytes((N, HQ, D), (N, HQ, D), (N, HKV, D), (N, HKV, D), (N, HKV, D),
                     (N, HKV, D), (N, D // 2), (N, D // 2))
    nope = _nbytes((N, HKV, D), (N, HKV, D), (N, HKV, D), (N, HKV, D))
    assert bench.rope_bytes(N) == rotate
    assert bench.rope_bytes(N, rotate=False) == nope


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    line = json.loads(r.stdout.strip().splitlines()[-1])
    assert "one GPU" in line["error"]
