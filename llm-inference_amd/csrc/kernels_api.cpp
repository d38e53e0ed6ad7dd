// Definitions of the reference's attention launch API (include/kernels/kernels.hpp)
// over the C ABI (include/attn_mi355x.h).  Behaviour follows the reference
// launchers: they return void and silently skip the shapes the reference skips
// (the C ABI returns 0 for those); a call the library rejects (arguments it
// cannot serve, or a failed kernel launch) throws std::runtime_error naming
// the launcher and the HIP error, so nothing fails silently.  The graph-node
// updaters exit through HIP_CHECK on failure, as the reference's do
// (causal_attention.hip.cpp:975-1026, rope.hip.cpp:208-241).
#include "../../include/kernels/kernels.hpp"

#include "../../include/attn_mi355x.h"
#include "../../include/gpu_utils.hpp"

#include <stdexcept>
#include <string>

namespace {

inline attn_f16_t* h(__half* p) { return reinterpret_cast<attn_f16_t*>(p); }
inline const attn_f16_t* h(const __half* p) { return reinterpret_cast<const attn_f16_t*>(p); }

// A non-zero C-ABI result: the launcher rejected its arguments or a kernel
// launch failed (the HIP runtime's last-error state is also set then).
inline void report(int rc, const char* launcher) {
    if (rc != 0)
        throw std::runtime_error(std::string("attn_mi355x: ") + launcher + " failed: " +
                                 hipGetErrorString((hipError_t)rc) + " (" +
                                 std::to_string(rc) + ")");
}

}  // namespace

void launch_qkv_gemm(const __half* d_input_norm, __half* d_qkv_out,
                     const __half* d_qkv_weights, const size_t seq_len,
                     const size_t hidden_size, const size_t total_qkv_dim) {
    report(attn_qkv_gemm(h(d_input_norm), h(d_qkv_out), h(d_qkv_weights), seq_len, hidden_size,
                         total_qkv_dim, nullptr), "launch_qkv_gemm");
}

void launch_qkv_gemm_rope_and_store_kv(const __half* d_input_norm, __half* d_qkv_out,
                                       const __half* d_qkv_weights, __half* d_k_cache,
                                       __half* d_v_cache, const __half* d_cos,
                                       const __half* d_sin, size_t seq_len, size_t hidden_size,
                                       size_t num_heads, size_t num_kv_heads, size_t head_dim,
                                       size_t start_pos, bool apply_rotation,
                                       hipStream_t stream) {
    report(attn_qkv_gemm_rope_store_kv(h(d_input_norm), h(d_qkv_out), h(d_qkv_weights),
                                       h(d_k_cache), h(d_v_cache), h(d_cos), h(d_sin), seq_len,
                                       hidden_size, num_heads, num_kv_heads, head_dim, start_pos,
                                       apply_rotation ? 1 : 0, stream),
           "launch_qkv_gemm_rope_and_store_kv");
}

void launch_qkv_decode(const __half* d_input_norm, __half* d_qkv_out,
                       const __half* d_qkv_weights, const size_t hidden_size,
                       const size_t total_qkv_dim, hipStream_t stream) {
    report(attn_qkv_decode(h(d_input_norm), h(d_qkv_out), h(d_qkv_weights), hidden_size,
                           total_qkv_dim, stream), "launch_qkv_decode");
}

void launch_qkv_rope_and_store_kv_decode(const __half* d_input_norm, __half* d_qkv_out,
                                         const __half* d_qkv_weights, __half* d_k_cache,
                                         __half* d_v_cache, const __half* d_cos,
                                         const __half* d_sin, size_t hidden_size,
                                         size_t num_heads, size_t num_kv_heads, size_t head_dim,
                                         size_t start_pos, bool apply_rotation,
                                         hipStream_t stream) {
    report(attn_qkv_rope_store_kv_decode(h(d_input_norm), h(d_qkv_out), h(d_qkv_weights),
                                         h(d_k_cache), h(d_v_cache), h(d_cos), h(d_sin),
                                         hidden_size, num_heads, num_kv_heads, head_dim,
                                         start_pos, apply_rotation ? 1 : 0, stream),
           "launch_qkv_rope_and_store_kv_decode");
}

void update_qkv_rope_and_store_kv_node(hipGraphExec_t graph_exec, hipGraphNode_t node,
                                       size_t start_pos, bool apply_rotation) {
    HIP_CHECK((hipError_t)attn_update_qkv_rope_node(graph_exec, node, start_pos,
                                                    apply_rotation ? 1 : 0));
}

void launch_attention_out_projection_decode(const __half* d_in, __half* d_out,
                                            const __half* d_o_proj_weights, size_t hidden_size,
                                            size_t num_heads, size_t head_dim, float beta,
                                            hipStream_t stream) {
    report(attn_out_proj_decode(h(d_in), h(d_out), h(d_o_proj_weights), hidden_size, num_heads,
                                head_dim, beta, stream), "launch_attention_out_projection_decode");
}

size_t decode_out_projection_workspace_bytes(size_t num_heads, size_t hidden_size) {
    return attn_decode_out_proj_workspace_bytes(num_heads, hidden_size);
}

void launch_causal_attention_decode_out_projection(
    const __half* d_q, const __half* d_k_cache, const __half* d_v_cache, __half* d_attn_out,
    float* d_partial_out, float* d_partial_max, float* d_partial_weight_sum, size_t kv_cache_len,
    size_t num_heads, size_t num_kv_heads, size_t head_dim, size_t kv_stride,
    const __half* d_o_proj_weights, __half* d_out, size_t hidden_size, float beta,
    void* d_workspace, hipStream_t stream, hipGraphNode_t* attention_node,
    hipGraphNode_t* merge_node) {
    const int rc = attn_decode_out_proj(
        h(d_q), h(d_k_cache), h(d_v_cache), h(d_attn_out), d_partial_out, d_partial_max,
        d_partial_weight_sum, kv_cache_len, num_heads, num_kv_heads, head_dim, kv_stride,
        h(d_o_proj_weights), h(d_out), hidden_size, beta, d_workspace, stream, attention_node,
        merge_node);
    report(rc, "launch_causal_attention_decode_out_projection");
}

void launch_rope(__half* d_q, __half* d_k, const __half* d_cos, const __half* d_sin,
                 size_t seq_len, size_t num_heads, size_t num_kv_heads, size_t head_dim,
                 size_t q_stride, size_t k_stride, size_t start_pos) {
    report(attn_rope(h(d_q), h(d_k), h(d_cos), h(d_sin), seq_len, num_heads, num_kv_heads,
                     head_dim, q_stride, k_stride, start_pos, nullptr), "launch_rope");
}

void launch_rope_and_store_kv(__half* d_q, __half* d_k, __half* d_v, __half* d_k_cache,
                              __half* d_v_cache, const __half* d_cos, const __half* d_sin,
                              size_t seq_len, size_t num_heads, size_t num_kv_heads,
                              size_t head_dim, size_t q_stride, size_t k_stride,
                              size_t start_pos, bool apply_rotation, hipStream_t stream) {
    report(attn_rope_store_kv(h(d_q), h(d_k), h(d_v), h(d_k_cache), h(d_v_cache), h(d_cos),
                              h(d_sin), seq_len, num_heads, num_kv_heads, head_dim, q_stride,
                              k_stride, start_pos, apply_rotation ? 1 : 0, stream),
           "launch_rope_and_store_kv");
}

void update_rope_and_store_kv_node(hipGraphExec_t graph_exec, hipGraphNode_t node,
                                   size_t start_pos, bool apply_rotation) {
    HIP_CHECK((hipError_t)attn_update_rope_node(graph_exec, node, start_pos,
                                                apply_rotation ? 1 : 0));
}

void launch_causal_attention_prefill(const __half* d_q, const __half* d_k, const __half* d_v,
                                     __half* d_out, size_t seq_len, size_t num_heads,
                                     size_t num_kv_heads, size_t head_dim, size_t q_stride,
                                     size_t kv_stride) {
    report(attn_prefill(h(d_q), h(d_k), h(d_v), h(d_out), seq_len, num_heads, num_kv_heads,
                        head_dim, q_stride, kv_stride, nullptr), "launch_causal_attention_prefill");
}

void launch_causal_attention_decode(const __half* d_q, const __half* d_k_cache,
                                    const __half* d_v_cache, __half* d_out, float* d_partial_out,
                                    float* d_partial_max, float* d_partial_weight_sum,
                                    size_t query_len, size_t kv_cache_len, size_t start_pos,
                                    size_t num_heads, size_t num_kv_heads, size_t head_dim,
                                    size_t q_stride, size_t kv_stride, hipStream_t stream,
                                    hipGraphNode_t* attention_node, hipGraphNode_t* merge_node) {
    const int rc = attn_decode(h(d_q), h(d_k_cache), h(d_v_cache), h(d_out), d_partial_out,
                               d_partial_max, d_partial_weight_sum, query_len, kv_cache_len,
                               start_pos, num_heads, num_kv_heads, head_dim, q_stride, kv_stride,
                               stream, attention_node, merge_node);
    // gpu_utils.hpp:45-59: a capture that does not end in exactly one node throws
    if (rc == (int)hipErrorIllegalState && (attention_node || merge_node))
        throw std::runtime_error("Expected one capture dependency");
    report(rc, "launch_causal_attention_decode");
}

void launch_causal_attention_decode_vectorized(
    const __half* d_q, const __half* d_k_cache, const __half* d_v_cache, __half* d_out,
    float* d_partial_out, float* d_partial_max, float* d_partial_weight_sum, size_t query_len,
    size_t kv_cache_len, size_t start_pos, size_t num_heads, size_t num_kv_heads,
    size_t head_dim, size_t q_stride, size_t kv_stride, hipStream_t stream,
    hipGraphNode_t* attention_node, hipGraphNode_t* merge_node) {
    // one decode implementation serves both reference entry points
    launch_causal_attention_decode(d_q, d_k_cache, d_v_cache, d_out, d_partial_out,
                                   d_partial_max, d_partial_weight_sum, query_len, kv_cache_len,
                                   start_pos, num_heads, num_kv_heads, head_dim, q_stride,
                                   kv_stride, stream, attention_node, merge_node);
}

void launch_rope_and_store_kv_decode(__half* d_q, const __half* d_k, const __half* d_v,
                                     __half* d_k_cache, __half* d_v_cache, const __half* d_cos,
                                     const __half* d_sin, __half* d_out, float* d_partial_out,
                                     float* d_partial_max, float* d_partial_weight_sum,
                                     size_t kv_cache_len, size_t start_pos, size_t num_heads,
                                     size_t num_kv_heads, size_t head_dim, bool apply_rotation,
                                     hipStream_t stream, hipGraphNode_t* attention_node,
                                     hipGraphNode_t* merge_node) {
    const int rc = attn_rope_store_kv_decode(
        h(d_q), h(d_k), h(d_v), h(d_k_cache), h(d_v_cache), h(d_cos), h(d_sin), h(d_out),
        d_partial_out, d_partial_max, d_partial_weight_sum, kv_cache_len, start_pos, num_heads,
        num_kv_heads, head_dim, 0, apply_rotation ? 1 : 0, stream, attention_node, merge_node);
    // gpu_utils.hpp:45-59: a capture that does not end in exactly one node throws
    if (rc == (int)hipErrorIllegalState && (attention_node || merge_node))
        throw std::runtime_error("Expected one capture dependency");
    report(rc, "launch_rope_and_store_kv_decode");
}

void update_rope_and_store_kv_decode_nodes(hipGraphExec_t graph_exec,
                                           hipGraphNode_t attention_node,
                                           hipGraphNode_t merge_node, size_t kv_cache_len,
                                           size_t start_pos, bool apply_rotation) {
    HIP_CHECK((hipError_t)attn_update_rope_decode_nodes(graph_exec, attention_node, merge_node,
                                                        kv_cache_len, start_pos,
                                                        apply_rotation ? 1 : 0));
}

void update_merge_attention_decode_node(hipGraphExec_t graph_exec, hipGraphNode_t node,
                                        size_t kv_cache_len) {
    HIP_CHECK((hipError_t)attn_update_merge_node(graph_exec, node, kv_cache_len));
}

void update_causal_attention_decode_node(hipGraphExec_t graph_exec, hipGraphNode_t node,
                                         size_t kv_cache_len) {
    HIP_CHECK((hipError_t)attn_update_decode_node(graph_exec, node, kv_cache_len));
}
