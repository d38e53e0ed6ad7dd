// The reference's QKV test chain (tests/test_qkv_gemm.cpp:26-119 of
// MarcVivas/llm-inference) on a model loaded through the reference-named
// headers: MemoryMappedFile + Model (weights.bin parsed, payload uploaded as
// DeviceWeights, RoPE tables built), then launch_qkv_gemm with a layer's
// q_proj as the fused QKV weight, launch_rope on the interleaved [N][3072]
// output, and launch_causal_attention_prefill reading Q/K/V from it with
// stride total_qkv_dim.
//
// usage: test_model_weights <weights.bin> <prefix> <seq_len> <layer>
// reads <prefix>.x (fp16 [seq_len][hidden_size]) and writes <prefix>.qkv (after
// the GEMM), <prefix>.rope (after RoPE) and <prefix>.attn (attention output),
// and prints the device offsets of the layer's tensors and the tokenizer JSON
// length for the caller to check.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <string>
#include <vector>

#include "gpu_utils.hpp"
#include "kernels/kernels.hpp"
#include "model.hpp"

static std::vector<__half> read_file(const std::string& path, size_t n) {
    std::vector<__half> v(n);
    std::ifstream f(path, std::ios::binary);
    f.read(reinterpret_cast<char*>(v.data()), std::streamsize(n * sizeof(__half)));
    if (!f) {
        std::fprintf(stderr, "cannot read %zu halves from %s\n", n, path.c_str());
        std::exit(2);
    }
    return v;
}

static void write_device(const std::string& path, const __half* d, size_t n) {
    std::vector<__half> h(n);
    HIP_CHECK(hipMemcpy(h.data(), d, n * sizeof(__half), hipMemcpyDeviceToHost));
    std::ofstream f(path, std::ios::binary);
    f.write(reinterpret_cast<const char*>(h.data()), std::streamsize(n * sizeof(__half)));
}

int main(int argc, char** argv) {
    if (argc != 5) {
        std::fprintf(stderr, "usage: %s <weights.bin> <prefix> <seq_len> <layer>\n", argv[0]);
        return 2;
    }
    const std::string prefix = argv[2];
    const size_t seq_len = std::strtoull(argv[3], nullptr, 10);
    const size_t layer = std::strtoull(argv[4], nullptr, 10);
    HIP_CHECK(hipSetDevice(0));

    MemoryMappedFile file(argv[1]);
    const Model model(file);
    const ModelConfig& c = model.config;
    if (layer >= c.num_layers) return 2;
    const size_t q_dim = size_t(c.num_heads) * c.head_dim;
    const size_t kv_dim = size_t(c.num_kv_heads) * c.head_dim;
    const size_t total_qkv_dim = q_dim + 2 * kv_dim;
    const TransformerBlock& block = model.device_weights.transformer_blocks[layer];
    const __half* base = model.device_weights.raw_device_buffer;
    std::printf("offsets %td %td %td %td %td\n", block.q_proj - base, block.k_proj - base,
                block.v_proj - base, block.o_proj - base, model.device_weights.lm_head - base);
    std::printf("tokenizer %zu\n", model.tokenizer_json.size());

    const std::vector<__half> x = read_file(prefix + ".x", seq_len * c.hidden_size);
    __half *d_x = nullptr, *d_qkv = nullptr, *d_attn = nullptr;
    HIP_CHECK(hipMalloc(&d_x, x.size() * sizeof(__half)));
    HIP_CHECK(hipMalloc(&d_qkv, seq_len * total_qkv_dim * sizeof(__half)));
    HIP_CHECK(hipMalloc(&d_attn, seq_len * q_dim * sizeof(__half)));
    HIP_CHECK(hipMemcpy(d_x, x.data(), x.size() * sizeof(__half), hipMemcpyHostToDevice));

    // test_qkv_gemm.cpp:50-59: q_proj is the start of the fused QKV weight
    launch_qkv_gemm(d_x, d_qkv, block.q_proj, seq_len, c.hidden_size, total_qkv_dim);
    HIP_CHECK(hipGetLastError());
    HIP_CHECK(hipDeviceSynchronize());
    write_device(prefix + ".qkv", d_qkv, seq_len * total_qkv_dim);

    // :91-94: RoPE in place on the interleaved output
    launch_rope(d_qkv, d_qkv + q_dim, model.rope_cache.d_cos, model.rope_cache.d_sin, seq_len,
                c.num_heads, c.num_kv_heads, c.head_dim, total_qkv_dim, total_qkv_dim);
    HIP_CHECK(hipGetLastError());
    HIP_CHECK(hipDeviceSynchronize());
    write_device(prefix + ".rope", d_qkv, seq_len * total_qkv_dim);

    // :108-112: prefill attention straight from the interleaved buffer
    launch_causal_attention_prefill(d_qkv, d_qkv + q_dim, d_qkv + q_dim + kv_dim, d_attn, seq_len,
                                    c.num_heads, c.num_kv_heads, c.head_dim, total_qkv_dim,
                                    total_qkv_dim);
    HIP_CHECK(hipGetLastError());
    HIP_CHECK(hipDeviceSynchronize());
    write_device(prefix + ".attn", d_attn, seq_len * q_dim);

    HIP_CHECK(hipFree(d_x));
    HIP_CHECK(hipFree(d_qkv));
    HIP_CHECK(hipFree(d_attn));
    std::printf("done\n");
    return 0;
}
