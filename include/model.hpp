// Model: a weights.bin loaded the way the reference engine loads it
// (include/model.hpp:10-101 of MarcVivas/llm-inference): the header parsed
// and checked, the tokenizer JSON located and skipped to the 64-byte aligned
// payload, the payload uploaded as DeviceWeights, and the RoPE tables built for
// max_seq_len.  The file is parsed by attn_weights_parse() of
// libattn_mi355x.so, in the reference's order of checks and with its
// exception texts.  The reference also builds a tokenizers-cpp Tokenizer from
// the JSON; this library has no tokenizer, so Model keeps the JSON text
// (tokenizer_json) for a caller that builds one.
#pragma once
#include <hip/hip_fp16.h>

#include <span>
#include <stdexcept>
#include <string>

#include "attn_mi355x.h"
#include "device_weights.hpp"
#include "memory_mapped_file.hpp"
#include "model_config.hpp"
#include "rope_cache.hpp"

struct Model {
    ModelConfig config;
    DeviceWeights device_weights;
    std::string tokenizer_json;
    RopeCache rope_cache;

    explicit Model(const MemoryMappedFile& file) {
        const std::span<const std::byte> bytes = file.bytes();
        config = ModelConfig(bytes);
        attn_weights_layout lay;
        const int rc = attn_weights_parse(bytes.data(), bytes.size(), bytes.size(), &lay);
        if (rc != 0) {
            const char* msg = attn_weights_error_string(rc);
            throw std::runtime_error(msg ? msg : "Invalid model file");
        }
        tokenizer_json.assign(reinterpret_cast<const char*>(bytes.data()) + lay.tokenizer_offset,
                              lay.tokenizer_bytes);
        device_weights = DeviceWeights(
            config, reinterpret_cast<const __half*>(bytes.data() + lay.weights_offset),
            lay.weights_bytes);
        rope_cache = create_rope_cache(config.max_seq_len, config.head_dim, config.rope_theta);
    }
};
