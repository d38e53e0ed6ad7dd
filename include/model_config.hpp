// ModelConfig: the 44-byte header of weights.bin, with the reference's field
// names, defaults, size and exception texts (include/model_config.hpp:9-55 of
// MarcVivas/llm-inference; written by python/export_weights.py:51-68).  The
// byte layout is attn_model_config of attn_mi355x.h.  print_model_config uses
// <cstdio> (no <print> in this toolchain's libstdc++).
#pragma once
#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <span>
#include <stdexcept>
#include <string_view>

#include "attn_mi355x.h"

#pragma pack(push, 1)
struct ModelConfig {
    char magic[4];
    uint32_t vocab_size = 49152;
    uint32_t hidden_size;
    uint32_t num_layers = 16;
    uint32_t num_heads = 32;
    uint32_t num_kv_heads = 8;
    uint32_t head_dim;
    uint32_t intermediate_size;
    uint32_t max_seq_len;

    float rms_norm_eps = 1e-6;
    float rope_theta = 1.0;

    ModelConfig() = default;

    ModelConfig(const std::span<const std::byte> bytes) { import_model_config(bytes); }

    // model_config.hpp:33-43: size check, raw copy, magic check
    void import_model_config(const std::span<const std::byte> bytes) {
        if (bytes.size() < sizeof(ModelConfig))
            throw std::runtime_error(attn_weights_error_string(ATTN_WEIGHTS_SHORT_HEADER));
        std::memcpy(static_cast<void*>(this), bytes.data(), sizeof(ModelConfig));
        if (std::string_view(magic, 4) != "QWEN")
            throw std::runtime_error(attn_weights_error_string(ATTN_WEIGHTS_BAD_MAGIC));
    }

    void print_model_config() const {
        std::printf("Architecture Hyperparameters:\n");
        std::printf("Layers: %u, Hidden Size: %u, Vocab: %u\n", num_layers, hidden_size,
                    vocab_size);
        std::printf("Maximum sequence length: %u\n", max_seq_len);
        std::printf("Heads (Q/KV): %u/%u, Head Dim: %u, \n", num_heads, num_kv_heads, head_dim);
        std::printf("Intermediate Size (SwiGLU): %u\n", intermediate_size);
        std::printf("Rope Theta: %g, RMSNorm Epsilon: %g\n", rope_theta, rms_norm_eps);
    }
};
static_assert(sizeof(ModelConfig) == 44);
static_assert(sizeof(ModelConfig) == sizeof(attn_model_config));
#pragma pack(pop)
