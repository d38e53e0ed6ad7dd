// FP16 KV cache with the reference's layout and bookkeeping
// (include/kv_cache.hpp:8-83 of MarcVivas/llm-inference):
//   one device buffer for all layers; layer l starts at l * 2*S*Hkv*D
//   elements, K first ([S][Hkv*D]), V at + S*Hkv*D; row t of KV head h is at
//   t*Hkv*D + h*D (the kv_stride the attention launchers receive).
// The constructor takes any config object exposing num_layers, max_seq_len,
// num_kv_heads and head_dim (the reference passes its ModelConfig).
//
// The KVCache interface, layout arithmetic and capacity error text follow
// include/kv_cache.hpp:8-82 of
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

#include <cstddef>
#include <stdexcept>
#include <string>

#include "gpu_utils.hpp"

class KVCache {
    __half* d_kv_buffer = nullptr;
    size_t num_layers_ = 0;
    size_t max_seq_len_ = 0;
    size_t num_kv_heads_ = 0;
    size_t head_dim_ = 0;
    size_t current_cache_len = 0;

  public:
    template <typename Config>
    explicit KVCache(const Config& config)
        : num_layers_(config.num_layers),
          max_seq_len_(config.max_seq_len),
          num_kv_heads_(config.num_kv_heads),
          head_dim_(config.head_dim) {
        HIP_CHECK(hipMalloc(&d_kv_buffer, compute_total_bytes()));
    }

    // Key pointer for layer l: base + l * layer_stride (kv_cache.hpp:20-26)
    [[nodiscard]] __half* get_k_cache(size_t layer_idx) noexcept {
        return d_kv_buffer + layer_idx * layer_stride();
    }
    [[nodiscard]] const __half* get_k_cache(size_t layer_idx) const noexcept {
        return d_kv_buffer + layer_idx * layer_stride();
    }
    // Value pointer for layer l: base + l * layer_stride + S * kv_dim (:28-34)
    [[nodiscard]] __half* get_v_cache(size_t layer_idx) noexcept {
        return d_kv_buffer + layer_idx * layer_stride() + max_seq_len_ * kv_dim();
    }
    [[nodiscard]] const __half* get_v_cache(size_t layer_idx) const noexcept {
        return d_kv_buffer + layer_idx * layer_stride() + max_seq_len_ * kv_dim();
    }

    size_t get_cached_len() const noexcept { return current_cache_len; }

    // kv_cache.hpp:40-45: throws past capacity
    void set_cached_len(size_t cached_len) {
        if (cached_len > max_seq_len_)
            throw std::out_of_range("KV cache capacity exceeded: requested " +
                                    std::to_string(cached_len) + " tokens, capacity " +
                                    std::to_string(max_seq_len_));
        current_cache_len = cached_len;
    }

    void reset_cache() { current_cache_len = 0; }

    ~KVCache() {
        if (d_kv_buffer) (void)hipFree(d_kv_buffer);
        d_kv_buffer = nullptr;
    }

    KVCache(const KVCache&) = delete;
    KVCache& operator=(const KVCache&) = delete;
    KVCache(KVCache&& o) noexcept
        : d_kv_buffer(o.d_kv_buffer),
          num_layers_(o.num_layers_),
          max_seq_len_(o.max_seq_len_),
          num_kv_heads_(o.num_kv_heads_),
          head_dim_(o.head_dim_),
          current_cache_len(o.current_cache_len) {
        o.d_kv_buffer = nullptr;
        o.current_cache_len = 0;
    }
    KVCache& operator=(KVCache&& o) = delete;

    // kv_cache.hpp:71-73
    size_t compute_total_bytes() const noexcept {
        return 2 * num_kv_heads_ * head_dim_ * max_seq_len_ * sizeof(__half) * num_layers_;
    }
    // kv_cache.hpp:76-82
    size_t kv_dim() const noexcept { return num_kv_heads_ * head_dim_; }
    size_t layer_stride() const noexcept { return 2 * num_kv_heads_ * head_dim_ * max_seq_len_; }
    size_t max_seq_len() const noexcept { return max_seq_len_; }
};
