// RoPE cos/sin tables with the reference's layout and arithmetic
// (include/rope_cache.hpp:9-105 of MarcVivas/llm-inference): fp16 tables
// [max_seq_len][head_dim/2], inv_freq[i] = 1/powf(theta, 2i/D),
// angle = float(pos) * inv_freq[i], cos/sin in fp32 rounded to fp16.  The
// host tables are produced by attn_rope_tables() of libattn_mi355x.so.
//
// The RopeCache holder and compute_inverse_frequencies follow
// include/rope_cache.hpp:9-60 of
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

#include <cmath>
#include <cstring>
#include <vector>

#include "attn_mi355x.h"
#include "gpu_utils.hpp"

struct RopeCache {
    __half* d_cos = nullptr;
    __half* d_sin = nullptr;

    ~RopeCache() {
        if (d_cos) HIP_CHECK(hipFree(d_cos));
        if (d_sin) HIP_CHECK(hipFree(d_sin));
    }

    RopeCache() = default;
    RopeCache(const RopeCache&) = delete;
    RopeCache& operator=(const RopeCache&) = delete;
    RopeCache(RopeCache&& o) noexcept : d_cos(o.d_cos), d_sin(o.d_sin) {
        o.d_cos = nullptr;
        o.d_sin = nullptr;
    }
    RopeCache& operator=(RopeCache&& o) noexcept {
        if (this != &o) {
            if (d_cos) HIP_CHECK(hipFree(d_cos));
            if (d_sin) HIP_CHECK(hipFree(d_sin));
            d_cos = o.d_cos;
            d_sin = o.d_sin;
            o.d_cos = nullptr;
            o.d_sin = nullptr;
        }
        return *this;
    }
};

// rope_cache.hpp:48-60
inline std::vector<float> compute_inverse_frequencies(size_t head_dim, float rope_theta) {
    const size_t half_dim = head_dim / 2;
    std::vector<float> inv_freq(half_dim);
    for (size_t i = 0; i < half_dim; ++i) {
        const float exponent = static_cast<float>(2 * i) / static_cast<float>(head_dim);
        inv_freq[i] = 1.0f / std::pow(rope_theta, exponent);
    }
    return inv_freq;
}

// rope_cache.hpp:78-105: tables computed on the host, uploaded once
inline RopeCache create_rope_cache(size_t max_seq_len, size_t head_dim, float rope_theta) {
    RopeCache cache;
    const size_t total_elements = max_seq_len * (head_dim / 2);
    const size_t total_bytes = total_elements * sizeof(__half);
    std::vector<attn_f16_t> host_cos(total_elements), host_sin(total_elements);
    HIP_CHECK((hipError_t)attn_rope_tables(host_cos.data(), host_sin.data(), max_seq_len,
                                           head_dim, rope_theta));
    HIP_CHECK(hipMalloc(&cache.d_cos, total_bytes));
    HIP_CHECK(hipMalloc(&cache.d_sin, total_bytes));
    HIP_CHECK(hipMemcpy(cache.d_cos, host_cos.data(), total_bytes, hipMemcpyHostToDevice));
    HIP_CHECK(hipMemcpy(cache.d_sin, host_sin.data(), total_bytes, hipMemcpyHostToDevice));
    return cache;
}
