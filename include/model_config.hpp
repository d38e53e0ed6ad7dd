// ModelConfig: the 44-byte header of weights.bin as written by
// python/export_weights.py:51-68 of MarcVivas/llm-inference (the field names,
// order and types are that file format; the byte layout is attn_model_config
// of attn_mi355x.h).  Parsing errors carry the texts of
// attn_weights_error_string.  The engine calls print_model_config
// (src/main.cpp), so the name is kept; its one-line summary is this build's.
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
    // a default-constructed config holds the reference's defaults
    // (model_config.hpp:14-24: 49152 vocab, 16 layers, 32 / 8 heads, eps 1e-6,
    // theta 1); the fields the reference leaves uninitialised start at zero
    char magic[4] = {};
    uint32_t vocab_size = 49152;
    uint32_t hidden_size = 0;
    uint32_t num_layers = 16;
    uint32_t num_heads = 32;
    uint32_t num_kv_heads = 8;
    uint32_t head_dim = 0;
    uint32_t intermediate_size = 0;
    uint32_t max_seq_len = 0;
    float rms_norm_eps = 1e-6f;
    float rope_theta = 1.0f;

    ModelConfig() = default;

    ModelConfig(const std::span<const std::byte> bytes) { import_model_config(bytes); }

    // the header is the first 44 bytes; its magic identifies the format
    void import_model_config(const std::span<const std::byte> bytes) {
        if (bytes.size() < sizeof(ModelConfig))
            throw std::runtime_error(attn_weights_error_string(ATTN_WEIGHTS_SHORT_HEADER));
        std::memcpy(static_cast<void*>(this), bytes.data(), sizeof(ModelConfig));
        if (std::string_view(magic, 4) != "QWEN")
            throw std::runtime_error(attn_weights_error_string(ATTN_WEIGHTS_BAD_MAGIC));
    }

    // one line: "<layers>L d<hidden> q<Hq>/kv<Hkv>x<head_dim> ffn<...> ..."
    void print_model_config() const {
        std::printf("weights.bin %.4s: %uL d%u q%u/kv%ux%u ffn%u vocab%u ctx%u theta=%g eps=%g\n",
                    magic, num_layers, hidden_size, num_heads, num_kv_heads, head_dim,
                    intermediate_size, vocab_size, max_seq_len, rope_theta, rms_norm_eps);
    }
};
static_assert(sizeof(ModelConfig) == 44);
static_assert(sizeof(ModelConfig) == sizeof(attn_model_config));
#pragma pack(pop)
