"""The C ABI without a GPU: the library loads, exports every entry point that
include/attn_mi355x.h declares, its host-side pieces (RoPE tables, workspace
sizing) match the oracle, and the reference's silent no-op shapes return 0
without touching a device.  CPU only."""
import ctypes
import pathlib
import re

import numpy as np
import pytest

import oracle

ROOT = pathlib.Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "attn_mi355x.h"


def declared_symbols():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(attn_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_reference_entry_points():
    names = declared_symbols()
    for n in ("attn_rope_store_kv", "attn_rope", "attn_update_rope_node", "attn_prefill",
              "attn_decode", "attn_update_decode_node", "attn_update_merge_node"):
        assert n in names


def test_library_exports_every_declared_symbol(attn):
    lib = attn.lib()
    missing = [n for n in declared_symbols() if not hasattr(lib, n)]
    assert not missing, missing
    assert sorted(attn.exported_symbols()) == declared_symbols()
    assert b"gfx950" in lib.attn_version()


def test_library_is_gfx950_code():
    so = (ROOT / "llm-inference_amd" / "lib" / "libattn_mi355x.so").read_bytes()
    assert b"gfx950" in so
    assert b"gfx942" not in so and b"gfx1030" not in so


@pytest.mark.parametrize("S,D,theta", [(300, 128, 5.0e6), (40000, 128, 5.0e6), (64, 32, 1.0e4)])
def test_host_rope_tables_bitexact_vs_oracle(attn, S, D, theta):
    c, s = attn.rope_tables(S, D, theta)
    oc, os_ = oracle.rope_tables(S, D, theta)
    assert np.array_equal(c.numpy().view(np.uint16), oc)
    assert np.array_equal(s.numpy().view(np.uint16), os_)


def test_workspace_states_formula(attn):
    # model_inference.hpp:192-198 and kernels.hpp:103 (KV_CHUNK = 12)
    for L in (1, 12, 13, 254, 32768, 32769):
        assert attn.decode_workspace_states(16, L) == 16 * ((L + 11) // 12)


def test_noop_shapes_touch_nothing(attn):
    lib = attn.lib()
    # launch_rope_and_store_kv: seq_len == 0 (rope.hip.cpp:156)
    assert lib.attn_rope_store_kv(None, None, None, None, None, None, None, 0, 16, 4, 128, 0, 0,
                                  0, 1, None) == 0
    # prefill: seq_len == 0, num_kv_heads == 0, Hq % Hkv != 0 (causal_attention.hip.cpp:392-399)
    for n, hq, hkv in ((0, 16, 4), (8, 16, 0), (8, 16, 3)):
        assert lib.attn_prefill(None, None, None, None, n, hq, hkv, 128, 0, 0, None) == 0
    # decode: query_len == 0, kv_len == 0, num_kv_heads == 0, head_dim == 0,
    # Hq % Hkv != 0 (:860-866, :945-946)
    for ql, L, hq, hkv, d in ((0, 5, 16, 4, 128), (1, 0, 16, 4, 128), (1, 5, 16, 0, 128),
                              (1, 5, 16, 4, 0), (1, 5, 16, 3, 128)):
        assert lib.attn_decode(None, None, None, None, None, None, None, ql, L, 0, hq, hkv, d, 0,
                               0, None, None, None) == 0
    # QKV projection with no output rows (matrix_vec_mul.hip.cpp:160)
    assert lib.attn_qkv_decode(None, None, None, 2048, 0, None) == 0
    assert lib.attn_qkv_rope_store_kv_decode(None, None, None, None, None, None, None, 2048, 0, 0,
                                             128, 0, 1, None) == 0
    # fused RoPE + decode: the no-op shapes of both launches it replaces
    for L, hq, hkv, d in ((0, 16, 4, 128), (5, 16, 0, 128), (5, 16, 4, 0), (5, 16, 3, 128)):
        assert lib.attn_rope_store_kv_decode(*([None] * 11), L, 0, hq, hkv, d, 0, 1, None, None,
                                             None) == 0


def test_invalid_arguments_are_errors(attn):
    lib = attn.lib()
    # odd head_dim cannot be split into rotation pairs
    assert lib.attn_rope_store_kv(None, None, None, None, None, None, None, 1, 16, 4, 127, 0, 0,
                                  0, 1, None) != 0
    # NoPE copy without a cache
    assert lib.attn_rope_store_kv(None, None, None, None, None, None, None, 1, 16, 4, 128, 0, 0,
                                  0, 0, None) != 0
    assert lib.attn_set_option(b"no_such_option", 1) == -1
    assert lib.attn_update_decode_node(None, None, 0) != 0
    # null data pointers are rejected before anything is launched
    assert lib.attn_prefill(None, None, None, None, 8, 16, 4, 128, 0, 0, None) != 0
    assert lib.attn_decode(None, None, None, None, None, None, None, 1, 5, 4, 16, 4, 128, 0, 0,
                           None, None, None) != 0
    # QKV projection: null output / operands, odd head_dim, missing caches or tables
    assert lib.attn_qkv_decode(None, None, None, 2048, 3072, None) != 0
    assert lib.attn_qkv_decode(None, 16, None, 2048, 3072, None) != 0
    y = 16
    assert lib.attn_qkv_rope_store_kv_decode(16, y, 16, 16, 16, 16, 16, 2048, 16, 4, 127, 0, 1,
                                             None) != 0
    assert lib.attn_qkv_rope_store_kv_decode(16, y, 16, None, 16, 16, 16, 2048, 16, 4, 128, 0, 1,
                                             None) != 0
    assert lib.attn_qkv_rope_store_kv_decode(16, y, 16, 16, 16, None, 16, 2048, 16, 4, 128, 0, 1,
                                             None) != 0
    assert lib.attn_update_qkv_rope_node(None, None, 0, 1) != 0
    # fused RoPE + decode: null pointers, missing tables when rotating; and,
    # when graph node handles are requested (the pair must be patchable), cache
    # rows not kv_dim apart or the new token outside the decoded range are
    # rejected with hipErrorInvalidValue before any HIP call
    p = [16] * 11
    an, mn = ctypes.c_void_p(), ctypes.c_void_p()
    def fused(ptrs, L=64, pos=63, kvs=0, apply=1, nodes=False):
        return lib.attn_rope_store_kv_decode(
            *ptrs, L, pos, 16, 4, 128, kvs, apply, None,
            ctypes.byref(an) if nodes else None, ctypes.byref(mn) if nodes else None)
    assert fused([None] + p[1:]) != 0
    assert fused(p[:5] + [None] + p[6:]) != 0
    assert fused(p, kvs=520, nodes=True) == 1  # hipErrorInvalidValue
    assert fused(p, pos=64, nodes=True) == 1
    assert fused([16] * 4 + [24] + [16] * 6, nodes=True) == 1  # a cache pointer not 16-byte aligned
    assert lib.attn_update_rope_decode_nodes(None, None, None, 64, 64, 1) != 0
    assert lib.attn_update_rope_decode_nodes(None, None, None, 0, 0, 1) != 0


def test_out_projection_host_rules(attn):
    """launch_attention_out_projection_decode and the decode + o_proj entry
    point: the no-op and error rules that need no GPU, and the workspace
    size (fp32 head partials rounded up to 256 bytes, then one uint32 counter
    per 128 output rows)."""
    lib = attn.lib()
    # hidden_size == 0 launches nothing, even with null pointers
    # (matrix_vec_mul.hip.cpp:160)
    assert lib.attn_out_proj_decode(None, None, None, 0, 16, 128, 1.0, None) == 0
    # null operands with a non-empty projection
    assert lib.attn_out_proj_decode(None, None, None, 2048, 16, 128, 1.0, None) != 0
    assert lib.attn_out_proj_decode(None, 16, None, 2048, 16, 128, 1.0, None) != 0
    # decode + o_proj with kv_len 0 and hidden 0: both replaced launches are no-ops
    assert lib.attn_decode_out_proj(*([None] * 7), 0, 16, 4, 128, 0, None, None, 0, 1.0, None,
                                    None, None, None) == 0
    for Hq, hidden in ((16, 2048), (16, 2000), (12, 100), (1, 1)):
        part = (Hq * hidden * 4 + 255) // 256 * 256
        assert lib.attn_decode_out_proj_workspace_bytes(Hq, hidden) == part + 4 * ((hidden + 127) // 128)


def test_decode_plan_respects_workspace_capacity(attn):
    # whatever the split plan, the partial states (one per split) fit in the
    # reference-sized workspace Hq * ceil(L / 12)
    lengths = (1, 2, 12, 13, 31, 32, 33, 63, 64, 65, 100, 129, 254, 255, 256, 257, 1000, 4096,
               32768, 65536, 131072)
    try:
        for splits in (0, 1, 2, 3, 64, 256, 1024):
            attn.set_option("decode_splits", splits)
            for L in lengths:
                for hq, hkv in ((16, 4), (4, 4), (2, 1), (16, 1), (32, 8), (8, 2)):
                    p = attn.decode_plan(L, hq, hkv, 128)
                    # one KV head per workgroup up to 12288 keys
                    hpw = 2 if hkv % 2 == 0 and L > 12288 else 1
                    assert p["path"] == {4: 1, 2: 2, 1: 3}[hpw]
                    assert attn.decode_hpw(p["path"]) == hpw
                    assert p["nsplit"] >= 1 and p["chunk"] * p["nsplit"] >= L
                    assert (p["nsplit"] - 1) * p["chunk"] < L  # no empty split
                    assert p["nstate"] == p["nsplit"]
                    assert hq * p["nstate"] <= hq * ((L + 11) // 12), (splits, L, hq, hkv, p)
    finally:
        attn.set_option("decode_splits", 0)
    # heads per workgroup can be forced within what Hkv allows
    try:
        for hpw, hkv, path in ((4, 4, 1), (4, 2, 2), (2, 4, 2), (1, 4, 3), (4, 1, 3)):
            attn.set_option("decode_heads_per_workgroup", hpw)
            assert attn.decode_plan(4096, 16, hkv, 128)["path"] == path, (hpw, hkv)
    finally:
        attn.set_option("decode_heads_per_workgroup", 0)
    # head_dim != 128 or an odd stride takes the generic kernel
    assert attn.decode_plan(257, 4, 2, 32)["path"] == 0
    assert attn.decode_plan(257, 4, 2, 128, kv_stride=2 * 128 + 17)["path"] == 0


def test_decode_plan_shapes(attn):
    """The planner's choices for the SmolLM3 decode shape (16 / 4 heads,
    D = 128, 256 CUs): one kernel (one split per KV head) up to 384 keys
    unless decode_whole_max_keys says otherwise; above, one KV head per
    workgroup and 64 splits up to 12288 keys; two KV heads per workgroup
    above, with chunks of at least 160 keys while that leaves fewer than 128
    splits."""
    p = lambda L: attn.decode_plan(L, 16, 4, 128)  # noqa: E731
    for L in (1, 16, 17, 100, 254, 384):
        assert p(L)["nsplit"] == 1 and p(L)["nstate"] == 1 and p(L)["path"] == 3, L
    assert p(385)["nsplit"] > 1
    try:
        attn.set_option("decode_whole_max_keys", -1)
        assert p(254)["nsplit"] == 16 and p(254)["chunk"] == 16
        attn.set_option("decode_whole_max_keys", 1000)
        assert p(1000)["nsplit"] == 1 and p(1001)["nsplit"] > 1
    finally:
        attn.set_option("decode_whole_max_keys", 0)
    # forced split counts or heads per workgroup keep the split plans
    try:
        attn.set_option("decode_heads_per_workgroup", 2)
        assert p(254)["nsplit"] > 1
    finally:
        attn.set_option("decode_heads_per_workgroup", 0)
    assert (p(4096)["path"], p(4096)["nsplit"], p(4096)["chunk"]) == (3, 64, 64)
    assert (p(16384)["path"], p(16384)["nsplit"], p(16384)["chunk"]) == (2, 103, 160)
    assert (p(32768)["path"], p(32768)["nsplit"], p(32768)["chunk"]) == (2, 128, 256)
    assert (p(65536)["path"], p(65536)["nsplit"], p(65536)["chunk"]) == (2, 128, 512)
    for L in range(12289, 20481, 256):
        assert p(L)["chunk"] >= 160 and p(L)["nsplit"] <= 128, (L, p(L))
    # no device work has been captured here: no node records
    assert attn.lib().attn_graph_node_records() == 0
    assert attn.lib().attn_set_option(b"graph_node_records", 0) == 0


def test_prefill_plan(attn):
    a = 4096
    assert attn.prefill_plan(a, a, a, a, 16, 4, 128, 3072, 512) == 1
    assert attn.prefill_plan(a, a, a, a, 16, 4, 64, 0, 0) == 0       # D != 128
    assert attn.prefill_plan(a, a, a, a, 16, 16, 128, 0, 0) == 0     # group of 1
    assert attn.prefill_plan(a, a, a, a, 16, 4, 128, 3075, 512) == 0  # unaligned stride
    assert attn.prefill_plan(a + 2, a, a, a, 16, 4, 128, 0, 0) == 0   # unaligned pointer
