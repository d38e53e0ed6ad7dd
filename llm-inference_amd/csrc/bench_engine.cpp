// Measurement helper for bench.py (libattn_bench.so): the reference engine's
// decode loop (model_inference.hpp:76-134 of MarcVivas/llm-inference)
// reduced to the attention path, driven through the reference's C++ launch
// API exactly as ModelInference drives it:
//  * the first token's layers are captured into one graph in global capture
//    mode (hipStreamCaptureModeGlobal, :96-101): per layer the RoPE + KV
//    append launch and the Flash-Decode launch, remembering the store_kv,
//    attention and merge nodes (enqueue_decode, :361-387);
//  * every later token patches each layer's three nodes with
//    update_rope_and_store_kv_node (start_pos, NoPE on every 4th layer),
//    update_causal_attention_decode_node and update_merge_attention_decode_node
//    (kv_len = start_pos + 1) (:105-123), launches the graph and synchronises
//    the stream (:126-130).
// With `fused` the layer is the fused RoPE + append + decode launch
// (launch_rope_and_store_kv_decode, one node) patched by
// update_rope_and_store_kv_decode_nodes.  Each layer's q/k/v come from its own
// row of `qkv` ([layers][Hq*D + 2*Hkv*D]); the per-token QKV producer is not
// part of this loop.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cstddef>
#include <vector>

#include "../../include/gpu_utils.hpp"
#include "../../include/kernels/kernels.hpp"

namespace {

double median(std::vector<double> v) {
    std::sort(v.begin(), v.end());
    return v.empty() ? 0.0 : v[v.size() / 2];
}

}  // namespace

extern "C" {

// cache: [layers][K|V][max_seq][Hkv*D]; positions first_pos .. first_pos +
// tokens - 1 are decoded (kv_len = position + 1 <= max_seq).  res[0..5]:
// median host patch us per token (the 3 * layers or layers updater calls),
// median per-token wall us (patch + launch + synchronize), median GPU us per
// token (events around the launch), capture + instantiate ms, min and max
// per-token wall us.  Returns 0 or a hipError_t.
int attn_bench_engine_decode(__half* cache, __half* qkv, const __half* cos, const __half* sin,
                             __half* out, float* part_out, float* part_max, float* part_sum,
                             size_t layers, size_t num_heads, size_t num_kv_heads,
                             size_t head_dim, size_t max_seq, size_t first_pos, size_t tokens,
                             int fused, double* res) {
    const size_t q_dim = num_heads * head_dim, kv_dim = num_kv_heads * head_dim;
    const size_t total = q_dim + 2 * kv_dim;
    if (!cache || !qkv || !cos || !sin || !out || !res || tokens < 2 ||
        first_pos + tokens > max_seq)
        return (int)hipErrorInvalidValue;
    struct Nodes { hipGraphNode_t store_kv = nullptr, attention = nullptr, merge = nullptr; };
    std::vector<Nodes> nodes(layers);
    hipStream_t stream = nullptr;
    if (hipError_t e = hipStreamCreateWithFlags(&stream, hipStreamNonBlocking)) return (int)e;
    auto k_cache = [&](size_t l) { return cache + l * 2 * max_seq * kv_dim; };
    auto v_cache = [&](size_t l) { return k_cache(l) + max_seq * kv_dim; };

    auto enqueue_decode = [&](size_t start_pos) {
        const size_t kv_len = start_pos + 1;
        for (size_t l = 0; l < layers; ++l) {
            __half* q = qkv + l * total;
            __half* k = q + q_dim;
            __half* v = k + kv_dim;
            const bool apply = (l + 1) % 4 != 0;  // model_inference.hpp:358
            if (fused) {
                launch_rope_and_store_kv_decode(q, k, v, k_cache(l), v_cache(l), cos, sin,
                                                out + l * q_dim, part_out, part_max, part_sum,
                                                kv_len, start_pos, num_heads, num_kv_heads,
                                                head_dim, apply, stream, &nodes[l].attention,
                                                &nodes[l].merge);
                continue;
            }
            launch_rope_and_store_kv(q, k, v, k_cache(l), v_cache(l), cos, sin, 1, num_heads,
                                     num_kv_heads, head_dim, total, total, start_pos, apply,
                                     stream);
            nodes[l].store_kv = last_captured_node(stream);
            launch_causal_attention_decode_vectorized(
                q, k_cache(l), v_cache(l), out + l * q_dim, part_out, part_max, part_sum, 1,
                kv_len, start_pos, num_heads, num_kv_heads, head_dim, total, kv_dim, stream,
                &nodes[l].attention, &nodes[l].merge);
        }
    };

    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    const auto c0 = std::chrono::steady_clock::now();
    HIP_CHECK(hipStreamBeginCapture(stream, hipStreamCaptureModeGlobal));
    enqueue_decode(first_pos);
    HIP_CHECK(hipStreamEndCapture(stream, &graph));
    HIP_CHECK(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0));
    const auto c1 = std::chrono::steady_clock::now();
    HIP_CHECK(hipGraphLaunch(exec, stream));
    HIP_CHECK(hipStreamSynchronize(stream));

    hipEvent_t e0, e1;
    HIP_CHECK(hipEventCreate(&e0));
    HIP_CHECK(hipEventCreate(&e1));
    std::vector<double> patch_us, wall_us, gpu_us;
    for (size_t t = 1; t < tokens; ++t) {
        const size_t start_pos = first_pos + t;
        const size_t kv_len = start_pos + 1;
        const auto t0 = std::chrono::steady_clock::now();
        for (size_t l = 0; l < layers; ++l) {
            const bool apply = (l + 1) % 4 != 0;
            if (fused) {
                update_rope_and_store_kv_decode_nodes(exec, nodes[l].attention, nodes[l].merge,
                                                      kv_len, start_pos, apply);
                continue;
            }
            update_rope_and_store_kv_node(exec, nodes[l].store_kv, start_pos, apply);
            update_causal_attention_decode_node(exec, nodes[l].attention, kv_len);
            update_merge_attention_decode_node(exec, nodes[l].merge, kv_len);
        }
        const auto t1 = std::chrono::steady_clock::now();
        HIP_CHECK(hipEventRecord(e0, stream));
        HIP_CHECK(hipGraphLaunch(exec, stream));
        HIP_CHECK(hipEventRecord(e1, stream));
        HIP_CHECK(hipStreamSynchronize(stream));
        const auto t2 = std::chrono::steady_clock::now();
        float ms = 0.f;
        HIP_CHECK(hipEventElapsedTime(&ms, e0, e1));
        patch_us.push_back(std::chrono::duration<double, std::micro>(t1 - t0).count());
        wall_us.push_back(std::chrono::duration<double, std::micro>(t2 - t0).count());
        gpu_us.push_back(ms * 1e3);
    }
    res[0] = median(patch_us);
    res[1] = median(wall_us);
    res[2] = median(gpu_us);
    res[3] = std::chrono::duration<double, std::milli>(c1 - c0).count();
    res[4] = *std::min_element(wall_us.begin(), wall_us.end());
    res[5] = *std::max_element(wall_us.begin(), wall_us.end());
    HIP_CHECK(hipEventDestroy(e0));
    HIP_CHECK(hipEventDestroy(e1));
    HIP_CHECK(hipGraphExecDestroy(exec));
    HIP_CHECK(hipGraphDestroy(graph));
    HIP_CHECK(hipStreamDestroy(stream));
    return 0;
}

}  // extern "C"
