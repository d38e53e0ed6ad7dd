// DeviceWeights / TransformerBlock: the model payload in one device allocation
// with per-tensor pointers, with the reference's members, constructor and
// move-only ownership (include/device_weights.hpp:9-154 of
// MarcVivas/llm-inference).  The pointer layout comes from
// attn_weights_layout_for() of libattn_mi355x.so, which is computed and
// checked before anything is allocated: a payload smaller than its header's
// tensors throws instead of handing out pointers past the allocation, and a
// payload with q_norm/k_norm per layer (written by the exporter for
// checkpoints that have them) sets q_norm/k_norm instead of shifting every
// later tensor.  q_proj is also the start of the fused [q_dim + 2*kv_dim][hidden]
// QKV weight (q_proj, k_proj, v_proj are adjacent).
//
// The DeviceWeights / TransformerBlock members, move semantics and
// exception texts follow include/device_weights.hpp:9-154 of
// MarcVivas/llm-inference, which is distributed under this notice:
//
//   MIT License
//
//   Copyright (c) 2026 MarcVivas
//
//   Permission is hereby granted, free of charge, to any person obtaining a copy
//   of this software and associated documentation files (the "Software"), to deal
//   in the Software without restriction, including without limitation the rights
//   to use, copy, modify, merge, publish, distribute, sublicense, and/or sell
//   copies of the Software, and to permit persons to whom the Software is
//   furnished to do so, subject to the following conditions:
//
//   The above copyright notice and this permission notice shall be included in all
//   copies or substantial portions of the Software.
//
//   THE SOFTWARE IS PROVIDED "AS IS", WITHOUT WARRANTY OF ANY KIND, EXPRESS OR
//   IMPLIED, INCLUDING BUT NOT LIMITED TO THE WARRANTIES OF MERCHANTABILITY,
//   FITNESS FOR A PARTICULAR PURPOSE AND NONINFRINGEMENT. IN NO EVENT SHALL THE
//   AUTHORS OR COPYRIGHT HOLDERS BE LIABLE FOR ANY CLAIM, DAMAGES OR OTHER
//   LIABILITY, WHETHER IN AN ACTION OF CONTRACT, TORT OR OTHERWISE, ARISING FROM,
//   OUT OF OR IN CONNECTION WITH THE SOFTWARE OR THE USE OR OTHER DEALINGS IN THE
//   SOFTWARE.
#pragma once
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "attn_mi355x.h"
#include "model_config.hpp"

struct TransformerBlock {
    const __half* input_normalization = nullptr;  // [hidden_size]
    const __half* q_proj = nullptr;               // [num_heads*head_dim][hidden_size]
    const __half* k_proj = nullptr;               // [num_kv_heads*head_dim][hidden_size]
    const __half* v_proj = nullptr;               // [num_kv_heads*head_dim][hidden_size]
    const __half* q_norm = nullptr;               // [head_dim] when present
    const __half* k_norm = nullptr;               // [head_dim] when present
    const __half* o_proj = nullptr;               // [hidden_size][num_heads*head_dim]
    const __half* post_attn_norm = nullptr;       // [hidden_size]
    const __half* gate_proj = nullptr;            // [intermediate_size][hidden_size]
    const __half* up_proj = nullptr;              // [intermediate_size][hidden_size]
    const __half* down_proj = nullptr;            // [hidden_size][intermediate_size]
};

struct DeviceWeights {
    __half* raw_device_buffer = nullptr;
    size_t total_bytes = 0;
    const __half* embedding_tokens = nullptr;  // [vocab_size][hidden_size]
    std::vector<TransformerBlock> transformer_blocks;
    const __half* final_norm = nullptr;        // [hidden_size]
    const __half* lm_head = nullptr;           // [vocab_size][hidden_size]

    DeviceWeights(const ModelConfig& config, const __half* host_weights, const size_t total_bytes) {
        attn_weights_layout lay;
        const int rc = attn_weights_layout_for(reinterpret_cast<const attn_model_config*>(&config),
                                               total_bytes, &lay);
        if (rc != 0) {
            const char* msg = attn_weights_error_string(rc);
            throw std::runtime_error(msg ? msg : "Invalid model weights");
        }
        hipError_t err = hipMalloc(&raw_device_buffer, total_bytes);
        if (err != hipSuccess) {
            raw_device_buffer = nullptr;
            throw std::runtime_error(std::string("Failed to allocate GPU memory: ") +
                                     hipGetErrorString(err));
        }
        this->total_bytes = total_bytes;
        err = hipMemcpy(raw_device_buffer, host_weights, total_bytes, hipMemcpyHostToDevice);
        if (err != hipSuccess) {
            release();
            throw std::runtime_error(std::string("Failed to copy weights to GPU: ") +
                                     hipGetErrorString(err));
        }
        const __half* base = raw_device_buffer;
        auto at = [base](uint64_t elems) -> const __half* { return base + elems; };
        auto opt = [&](uint64_t layer0, uint64_t rel) -> const __half* {
            return rel == UINT64_MAX ? nullptr : at(layer0 + rel);
        };
        embedding_tokens = at(lay.embedding);
        transformer_blocks.resize(config.num_layers);
        for (size_t i = 0; i < config.num_layers; ++i) {
            const uint64_t l0 = lay.layer_base + i * lay.layer_elems;
            TransformerBlock& b = transformer_blocks[i];
            b.input_normalization = at(l0 + lay.input_norm);
            b.q_proj = at(l0 + lay.q_proj);
            b.k_proj = at(l0 + lay.k_proj);
            b.v_proj = at(l0 + lay.v_proj);
            b.q_norm = opt(l0, lay.q_norm);
            b.k_norm = opt(l0, lay.k_norm);
            b.o_proj = at(l0 + lay.o_proj);
            b.post_attn_norm = at(l0 + lay.post_attn_norm);
            b.gate_proj = at(l0 + lay.gate_proj);
            b.up_proj = at(l0 + lay.up_proj);
            b.down_proj = at(l0 + lay.down_proj);
        }
        final_norm = at(lay.final_norm);
        lm_head = at(lay.lm_head);
    }

    ~DeviceWeights() { release(); }

    DeviceWeights() = default;
    DeviceWeights(const DeviceWeights&) = delete;
    DeviceWeights& operator=(const DeviceWeights&) = delete;

    DeviceWeights(DeviceWeights&& o) noexcept
        : raw_device_buffer(o.raw_device_buffer), total_bytes(o.total_bytes),
          embedding_tokens(o.embedding_tokens),
          transformer_blocks(std::move(o.transformer_blocks)), final_norm(o.final_norm),
          lm_head(o.lm_head) {
        o.raw_device_buffer = nullptr;
        o.total_bytes = 0;
    }

    DeviceWeights& operator=(DeviceWeights&& o) noexcept {
        if (this != &o) {
            release();
            raw_device_buffer = o.raw_device_buffer;
            total_bytes = o.total_bytes;
            embedding_tokens = o.embedding_tokens;
            transformer_blocks = std::move(o.transformer_blocks);
            final_norm = o.final_norm;
            lm_head = o.lm_head;
            o.raw_device_buffer = nullptr;
            o.total_bytes = 0;
        }
        return *this;
    }

private:
    void release() noexcept {
        if (raw_device_buffer) (void)hipFree(raw_device_buffer);
        raw_device_buffer = nullptr;
        total_bytes = 0;
    }
};
