"""The reference's C++ launch API (include/kernels/kernels.hpp) as exported by
libattn_mi355x.so.  CPU part: every function the header declares is defined in
the library with the reference's exact signature (checked through the
demangled names), and the reference-layout headers (kv_cache.hpp,
rope_cache.hpp, gpu_utils.hpp) compile as C++23 (the engine's standard) and
as C++17.  GPU part: the C++ test
program tests/cpp/test_reference_api.cpp, built against the library, runs the
reference-style checks (decode KAT, RoPE/KV append, decode vs prefill rows,
graph-captured multi-layer decode with node patching, the fused QKV and
RoPE + decode launchers against the reference's launch sequences)."""
import pathlib
import re
import subprocess

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
LIB = ROOT / "llm-inference_amd" / "lib" / "libattn_mi355x.so"
BIN = ROOT / "tests" / "cpp" / "_build" / "test_reference_api"
HIPCC = "/opt/rocm/bin/hipcc"

# kernels.hpp signatures of the reference (include/kernels/kernels.hpp:38-146),
# plus the fused decode-step producer, as the C++ demangler prints them
EXPECTED = {
    "launch_rope(__half*, __half*, __half const*, __half const*, unsigned long, unsigned long, "
    "unsigned long, unsigned long, unsigned long, unsigned long, unsigned long)",
    "launch_rope_and_store_kv(__half*, __half*, __half*, __half*, __half*, __half const*, "
    "__half const*, unsigned long, unsigned long, unsigned long, unsigned long, unsigned long, "
    "unsigned long, unsigned long, bool, ihipStream_t*)",
    "update_rope_and_store_kv_node(hipGraphExec*, hipGraphNode*, unsigned long, bool)",
    "launch_causal_attention_prefill(__half const*, __half const*, __half const*, __half*, "
    "unsigned long, unsigned long, unsigned long, unsigned long, unsigned long, unsigned long)",
    "launch_causal_attention_decode(__half const*, __half const*, __half const*, __half*, float*, "
    "float*, float*, unsigned long, unsigned long, unsigned long, unsigned long, unsigned long, "
    "unsigned long, unsigned long, unsigned long, ihipStream_t*, hipGraphNode**, hipGraphNode**)",
    "launch_causal_attention_decode_vectorized(__half const*, __half const*, __half const*, "
    "__half*, float*, float*, float*, unsigned long, unsigned long, unsigned long, unsigned long, "
    "unsigned long, unsigned long, unsigned long, unsigned long, ihipStream_t*, hipGraphNode**, "
    "hipGraphNode**)",
    "update_merge_attention_decode_node(hipGraphExec*, hipGraphNode*, unsigned long)",
    "update_causal_attention_decode_node(hipGraphExec*, hipGraphNode*, unsigned long)",
    "launch_qkv_decode(__half const*, __half*, __half const*, unsigned long, unsigned long, "
    "ihipStream_t*)",
    "launch_qkv_gemm(__half const*, __half*, __half const*, unsigned long, unsigned long, "
    "unsigned long)",
    "launch_qkv_gemm_rope_and_store_kv(__half const*, __half*, __half const*, __half*, __half*, "
    "__half const*, __half const*, unsigned long, unsigned long, unsigned long, unsigned long, "
    "unsigned long, unsigned long, bool, ihipStream_t*)",
    # fused decode-step producer (no reference counterpart)
    "launch_qkv_rope_and_store_kv_decode(__half const*, __half*, __half const*, __half*, __half*, "
    "__half const*, __half const*, unsigned long, unsigned long, unsigned long, unsigned long, "
    "unsigned long, bool, ihipStream_t*)",
    "update_qkv_rope_and_store_kv_node(hipGraphExec*, hipGraphNode*, unsigned long, bool)",
    # fused RoPE + decode (no reference counterpart)
    "launch_rope_and_store_kv_decode(__half*, __half const*, __half const*, __half*, __half*, "
    "__half const*, __half const*, __half*, float*, float*, float*, unsigned long, unsigned long, "
    "unsigned long, unsigned long, unsigned long, bool, ihipStream_t*, hipGraphNode**, "
    "hipGraphNode**)",
    "update_rope_and_store_kv_decode_nodes(hipGraphExec*, hipGraphNode*, hipGraphNode*, "
    "unsigned long, unsigned long, bool)",
    # kernels.hpp:179-187 of the reference, the decode step's consumer
    "launch_attention_out_projection_decode(__half const*, __half*, __half const*, "
    "unsigned long, unsigned long, unsigned long, float, ihipStream_t*)",
    # decode with its merge fused into o_proj (no reference counterpart)
    "launch_causal_attention_decode_out_projection(__half const*, __half const*, __half const*, "
    "__half*, float*, float*, float*, unsigned long, unsigned long, unsigned long, unsigned long, "
    "unsigned long, __half const*, __half*, unsigned long, float, void*, ihipStream_t*, "
    "hipGraphNode**, hipGraphNode**)",
}


def _exported_cpp_functions():
    out = subprocess.run(["nm", "-D", "--defined-only", "-C", str(LIB)], check=True,
                         capture_output=True, text=True).stdout
    names = set()
    for line in out.splitlines():
        parts = line.split(" ", 2)
        if len(parts) == 3 and parts[1] == "T" and "(" in parts[2]:
            names.add(parts[2])
    return names


def test_header_declares_exactly_the_hot_path_subset():
    text = (ROOT / "include" / "kernels" / "kernels.hpp").read_text()
    declared = set(re.findall(r"^void\s+(\w+)\s*\(", text, flags=re.M))
    assert declared == {sig.split("(")[0] for sig in EXPECTED}
    assert re.search(r"#define\s+KV_CHUNK\s+12\b", text)


def test_library_defines_every_reference_launcher(attn):
    exported = _exported_cpp_functions()
    missing = sorted(EXPECTED - exported)
    assert not missing, missing
    assert "decode_out_projection_workspace_bytes(unsigned long, unsigned long)" in exported


@pytest.mark.parametrize("std", ["c++17", "c++23"])
def test_reference_headers_compile(tmp_path, std):
    """The engine (model_inference.hpp) is C++23; the headers also stay valid
    C++17 for other callers."""
    src = tmp_path / "use_headers.cpp"
    src.write_text(
        '#include "kernels/kernels.hpp"\n#include "kv_cache.hpp"\n#include "rope_cache.hpp"\n'
        "struct Cfg { size_t num_layers = 2, max_seq_len = 8, num_kv_heads = 4, head_dim = 128; };\n"
        "static_assert(KV_CHUNK == 12);\n"
        "size_t f() { KVCache c{Cfg{}}; return c.layer_stride() + c.kv_dim(); }\n"
        "std::vector<float> g() { return compute_inverse_frequencies(128, 5.0e6f); }\n")
    r = subprocess.run([HIPCC, f"-std={std}", "-fsyntax-only", "-I", str(ROOT / "include"), str(src)],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr


@pytest.mark.parametrize("call", [
    "update_rope_and_store_kv_node(nullptr, nullptr, 5, true)",
    "update_causal_attention_decode_node(nullptr, nullptr, 5)",
    "update_merge_attention_decode_node(nullptr, nullptr, 5)",
    "update_qkv_rope_and_store_kv_node(nullptr, nullptr, 5, true)",
    "update_rope_and_store_kv_decode_nodes(nullptr, nullptr, nullptr, 5, 4, true)",
])
def test_node_updaters_exit_through_hip_check(tmp_path, call):
    """The reference's updaters wrap hipGraphExecKernelNodeSetParams in
    HIP_CHECK (causal_attention.hip.cpp:975-1026, rope.hip.cpp:208-241): a
    failure prints the HIP error and exits with status 1.  A node that cannot
    be read (here a null node, on any machine) takes that path."""
    src = tmp_path / "updater_failure.cpp"
    src.write_text('#include "kernels/kernels.hpp"\n#include <cstdio>\n'
                   f"int main() {{ {call}; std::puts(\"returned\"); return 0; }}\n")
    exe = tmp_path / "updater_failure"
    lib_dir = ROOT / "llm-inference_amd" / "lib"
    r = subprocess.run([HIPCC, "-std=c++23", "-I", str(ROOT / "include"), str(src), "-o", str(exe),
                        "-L", str(lib_dir), "-lattn_mi355x", f"-Wl,-rpath,{lib_dir}"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert r.returncode == 1, (r.returncode, r.stdout, r.stderr)
    assert "returned" not in r.stdout
    assert "[HIP Error]" in r.stderr


def test_rejected_launch_throws(tmp_path):
    """A launch the library cannot serve is not silent: the launcher throws
    std::runtime_error naming itself and the HIP error.  Null buffers with a
    non-empty shape are rejected before any HIP call, so this runs anywhere."""
    src = tmp_path / "rejected.cpp"
    src.write_text('#include "kernels/kernels.hpp"\n#include <cstdio>\n#include <stdexcept>\n'
                   "int main() {\n"
                   "  try { launch_qkv_decode(nullptr, nullptr, nullptr, 2048, 3072); }\n"
                   "  catch (const std::runtime_error& e) { std::puts(e.what()); return 3; }\n"
                   "  std::puts(\"returned\"); return 0;\n}\n")
    exe = tmp_path / "rejected"
    lib_dir = ROOT / "llm-inference_amd" / "lib"
    r = subprocess.run([HIPCC, "-std=c++23", "-I", str(ROOT / "include"), str(src), "-o", str(exe),
                        "-L", str(lib_dir), "-lattn_mi355x", f"-Wl,-rpath,{lib_dir}"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert r.returncode == 3, (r.returncode, r.stdout, r.stderr)
    assert "launch_qkv_decode failed" in r.stdout and "returned" not in r.stdout


@pytest.mark.gpu
def test_cpp_reference_api_program(gpu):
    assert BIN.exists(), f"{BIN} not built: run __graft_entry__.build()"
    r = subprocess.run([str(BIN)], capture_output=True, text=True, timeout=300)
    print(r.stdout)
    print(r.stderr)
    lines = [l for l in r.stdout.splitlines() if l.startswith(("PASS", "FAIL"))]
    assert len(lines) == 10, r.stdout + r.stderr
    assert r.returncode == 0, r.stdout + r.stderr


@pytest.mark.gpu
def test_cpp_engine_order_first_decode_inside_global_capture(gpu):
    """tests/cpp/test_engine_order.cpp in a process of its own: a prefill, then
    the process's first decode call made inside a hipStreamCaptureModeGlobal
    capture (model_inference.hpp:96-101), the graph launched, the next token
    patched through the three updaters per layer and launched again; each token
    equals eager launches bit for bit and an fp64 CPU attention."""
    exe = ROOT / "tests" / "cpp" / "_build" / "test_engine_order"
    assert exe.exists(), f"{exe} not built: run __graft_entry__.build()"
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    print(r.stdout)
    print(r.stderr)
    lines = [l for l in r.stdout.splitlines() if l.startswith(("PASS", "FAIL"))]
    assert len(lines) == 6, r.stdout + r.stderr
    assert r.returncode == 0, r.stdout + r.stderr
