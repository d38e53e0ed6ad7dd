// Attention hot-path launch API, declared exactly as in the reference's
// include/kernels/kernels.hpp (same names, parameter types, order and default
// arguments), so ModelInference (model_inference.hpp) and the reference tests
// compile unchanged against it.  Definitions live in
// llm-inference_amd/csrc/kernels_api.cpp (libattn_mi355x.so) and forward to the
// C ABI in include/attn_mi355x.h.  Only the attention subset is declared here;
// the GEMM/GEMV/norm/embedding launchers of the reference are outside this
// library.
//
// The declarations (names, parameter lists, default arguments) follow
// include/kernels/kernels.hpp:47-194 of
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
#include <cstdint>
#include <cstddef>
#include <hip/hip_runtime.h>

// kernels.hpp:29-36 (Y[seq][total] = X[seq][hidden] . W^T; no stream argument:
// the null stream, as the reference's rocBLAS handle uses)
void launch_qkv_gemm(
    const __half* d_input_norm,
    __half* d_qkv_out,
    const __half* d_qkv_weights,
    const size_t seq_len,
    const size_t hidden_size,
    const size_t total_qkv_dim
);

// kernels.hpp:38-45 (fp16 GEMV y = W x; W row-major [total_qkv_dim][hidden])
void launch_qkv_decode(
    const __half* d_input_norm,
    __half* d_qkv_out,
    const __half* d_qkv_weights,
    const size_t hidden_size,
    const size_t total_qkv_dim,
    hipStream_t stream = nullptr
);

// kernels.hpp:47-59
void launch_rope(
    __half* d_q,                 // [seq_len, num_heads, head_dim]
    __half* d_k,                 // [seq_len, num_kv_heads, head_dim]
    const __half* d_cos,         // [max_seq_len, head_dim / 2]
    const __half* d_sin,         // [max_seq_len, head_dim / 2]
    size_t seq_len,
    size_t num_heads,
    size_t num_kv_heads,
    size_t head_dim,
    size_t q_stride,
    size_t k_stride,
    size_t start_pos = 0         // Position offset (0 for prefill)
);

// kernels.hpp:62-79
void launch_rope_and_store_kv(
    __half* d_q,                 // [seq_len, num_heads, head_dim]
    __half* d_k,                 // [seq_len, num_kv_heads, head_dim]
    __half* d_v,                 // [seq_len, num_kv_heads, head_dim]
    __half* d_k_cache,           // [max_seq_len, num_kv_heads, head_dim]
    __half* d_v_cache,           // [max_seq_len, num_kv_heads, head_dim]
    const __half* d_cos,         // [max_seq_len, head_dim / 2]
    const __half* d_sin,         // [max_seq_len, head_dim / 2]
    size_t seq_len,
    size_t num_heads,
    size_t num_kv_heads,
    size_t head_dim,
    size_t q_stride,
    size_t k_stride,
    size_t start_pos,            // Position offset (0 for prefill)
    bool apply_rotation,
    hipStream_t stream = nullptr
);

// kernels.hpp:81-86
void update_rope_and_store_kv_node(
    hipGraphExec_t graph_exec,
    hipGraphNode_t node,
    size_t start_pos,
    bool apply_rotation
);

// kernels.hpp:88-99 (launched on the null stream, as in the reference)
void launch_causal_attention_prefill(
    const __half* d_q,
    const __half* d_k,
    const __half* d_v,
    __half* d_out,
    size_t seq_len,
    size_t num_heads,
    size_t num_kv_heads,
    size_t head_dim,
    size_t q_stride = 0,  // Elements between tokens; 0 means packed Q.
    size_t kv_stride = 0  // Elements between tokens; 0 means packed K/V.
);

// kernels.hpp:103: workspace sizing unit (tokens per partial state)
#define KV_CHUNK 12

// kernels.hpp:104-123
void launch_causal_attention_decode(
    const __half* d_q,              // [1, num_heads, head_dim]
    const __half* d_k_cache,        // [kv_cache_len, num_kv_heads, head_dim]
    const __half* d_v_cache,        // [kv_cache_len, num_kv_heads, head_dim]
    __half* d_out,                  // [1, num_heads, head_dim]
    float* d_partial_out,           // [num_heads, num_kv_chunks, head_dim]
    float* d_partial_max,           // [num_heads, num_kv_chunks]
    float* d_partial_weight_sum,    // [num_heads, num_kv_chunks]
    size_t query_len,               // Must be 1 for this decode implementation.
    size_t kv_cache_len,            // Number of valid cached tokens.
    size_t start_pos,               // Absolute position of the query token.
    size_t num_heads,
    size_t num_kv_heads,
    size_t head_dim,
    size_t q_stride,                // Elements between Q tokens; 0 means packed.
    size_t kv_stride,               // Elements between K/V tokens; 0 means packed.
    hipStream_t stream = nullptr,
    hipGraphNode_t* attention_node = nullptr,
    hipGraphNode_t* merge_node = nullptr
);

// kernels.hpp:127-146
void launch_causal_attention_decode_vectorized(
    const __half* d_q,
    const __half* d_k_cache,
    const __half* d_v_cache,
    __half* d_out,
    float* d_partial_out,
    float* d_partial_max,
    float* d_partial_weight_sum,
    size_t query_len,
    size_t kv_cache_len,
    size_t start_pos,
    size_t num_heads,
    size_t num_kv_heads,
    size_t head_dim,
    size_t q_stride = 0,
    size_t kv_stride = 0,
    hipStream_t stream = nullptr,
    hipGraphNode_t* attention_node = nullptr,
    hipGraphNode_t* merge_node = nullptr
);

// kernels.hpp:148-152
void update_merge_attention_decode_node(
    hipGraphExec_t graph_exec,
    hipGraphNode_t node,
    size_t kv_cache_len
);

// kernels.hpp:190-194
void update_causal_attention_decode_node(
    hipGraphExec_t graph_exec,
    hipGraphNode_t node,
    size_t kv_cache_len
);

// kernels.hpp:179-187: y = W_o x + beta * y (beta = 1 adds the residual).
void launch_attention_out_projection_decode(
    const __half* d_in,               // [num_heads * head_dim]
    __half* d_out,                    // [hidden_size]: residual in, projection out
    const __half* d_o_proj_weights,   // [hidden_size][num_heads * head_dim]
    size_t hidden_size,
    size_t num_heads,
    size_t head_dim,
    float beta,
    hipStream_t stream = nullptr
);

// Not in the reference: launch_causal_attention_decode_vectorized (query_len
// 1, start_pos kv_cache_len - 1) followed by
// launch_attention_out_projection_decode(d_attn_out, d_out, d_o_proj_weights,
// hidden_size, num_heads, head_dim, beta) (model_inference.hpp:371-397), as
// those launches; with the library option decode_out_proj_fused = 1 the
// decode's merge and the projection run as one kernel (measured slower on
// MI355X): *attention_node is the split kernel, *merge_node the merge (or
// fused) kernel, both patched by the existing updaters.  d_attn_out receives
// the attention output either way.  d_workspace:
// decode_out_projection_workspace_bytes(num_heads, hidden_size) bytes,
// zero-filled once before the first call (calls leave it reusable); calls
// sharing it must be ordered on one stream.  Shapes off the fused path issue
// the two launches.
size_t decode_out_projection_workspace_bytes(size_t num_heads, size_t hidden_size);
void launch_causal_attention_decode_out_projection(
    const __half* d_q,
    const __half* d_k_cache,
    const __half* d_v_cache,
    __half* d_attn_out,
    float* d_partial_out,
    float* d_partial_max,
    float* d_partial_weight_sum,
    size_t kv_cache_len,
    size_t num_heads,
    size_t num_kv_heads,
    size_t head_dim,
    size_t kv_stride,
    const __half* d_o_proj_weights,
    __half* d_out,
    size_t hidden_size,
    float beta,
    void* d_workspace,
    hipStream_t stream = nullptr,
    hipGraphNode_t* attention_node = nullptr,
    hipGraphNode_t* merge_node = nullptr
);

// Not in the reference: launch_qkv_decode followed by launch_rope_and_store_kv
// for one decode token (model_inference.hpp:354-369), fused into one kernel
// with identical results; d_qkv_out receives Q rotated, K and V as projected.
void launch_qkv_rope_and_store_kv_decode(
    const __half* d_input_norm,
    __half* d_qkv_out,
    const __half* d_qkv_weights,
    __half* d_k_cache,
    __half* d_v_cache,
    const __half* d_cos,
    const __half* d_sin,
    size_t hidden_size,
    size_t num_heads,
    size_t num_kv_heads,
    size_t head_dim,
    size_t start_pos,
    bool apply_rotation,
    hipStream_t stream = nullptr
);

// Not in the reference: patches start_pos / apply_rotation of a captured
// launch_qkv_rope_and_store_kv_decode node (cf. update_rope_and_store_kv_node).
void update_qkv_rope_and_store_kv_node(
    hipGraphExec_t graph_exec,
    hipGraphNode_t node,
    size_t start_pos,
    bool apply_rotation
);

// Not in the reference: launch_rope_and_store_kv for the decode token
// followed by launch_causal_attention_decode (model_inference.hpp:96-126) as
// the decode's two kernels (split, merge) with identical results: q is left
// rotated in place, the new K/V row appended at start_pos, d_out holds the
// attention.  Serves head_dim 128, 16-byte aligned tensors and start_pos <
// kv_cache_len; other shapes issue the two reference launches when no node
// handles are requested, and throw std::runtime_error (nothing enqueued) when
// they are, since update_rope_and_store_kv_decode_nodes patches only the
// fused pair.
void launch_rope_and_store_kv_decode(
    __half* d_q,
    const __half* d_k,
    const __half* d_v,
    __half* d_k_cache,
    __half* d_v_cache,
    const __half* d_cos,
    const __half* d_sin,
    __half* d_out,
    float* d_partial_out,
    float* d_partial_max,
    float* d_partial_weight_sum,
    size_t kv_cache_len,
    size_t start_pos,
    size_t num_heads,
    size_t num_kv_heads,
    size_t head_dim,
    bool apply_rotation,
    hipStream_t stream = nullptr,
    hipGraphNode_t* attention_node = nullptr,
    hipGraphNode_t* merge_node = nullptr
);

// Not in the reference: patches both captured nodes of
// launch_rope_and_store_kv_decode (cf. update_rope_and_store_kv_node and the
// two decode node updaters).
void update_rope_and_store_kv_decode_nodes(
    hipGraphExec_t graph_exec,
    hipGraphNode_t attention_node,
    hipGraphNode_t merge_node,
    size_t kv_cache_len,
    size_t start_pos,
    bool apply_rotation
);

// Not in the reference: launch_qkv_gemm followed by launch_rope_and_store_kv
// for a prefill of seq_len tokens (model_inference.hpp:266-285), fused into
// one kernel (head_dim 128) with identical results.
void launch_qkv_gemm_rope_and_store_kv(
    const __half* d_input_norm,
    __half* d_qkv_out,
    const __half* d_qkv_weights,
    __half* d_k_cache,
    __half* d_v_cache,
    const __half* d_cos,
    const __half* d_sin,
    size_t seq_len,
    size_t hidden_size,
    size_t num_heads,
    size_t num_kv_heads,
    size_t head_dim,
    size_t start_pos,
    bool apply_rotation,
    hipStream_t stream = nullptr
);
