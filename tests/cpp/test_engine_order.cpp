// The reference engine's call order in a fresh process (model_inference.hpp:
// 40-134): a prompt is prefilled (RoPE + KV append, causal prefill per layer,
// null stream), then the FIRST decode call of the process is made inside a
// hipStreamCaptureModeGlobal capture on a non-blocking stream (:96-101), so
// whatever the library does on its first decode (plan, device queries) runs
// under global capture.  The graph is instantiated and launched; then, for the
// next token, every layer's store_kv / attention / merge nodes are patched
// (:105-123) and the graph launched again.  Each token's outputs, rotated q and
// appended cache rows must equal the same launches issued eagerly on a copy,
// bit for bit, and the outputs must match an fp64 CPU attention over the
// cache (2e-3 + 1e-2 |e|).  Run as its own process; prints PASS/FAIL lines and
// exits with the number of failures.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <random>
#include <vector>

#include "../../include/gpu_utils.hpp"
#include "../../include/kernels/kernels.hpp"
#include "../../include/kv_cache.hpp"
#include "../../include/rope_cache.hpp"

namespace {

constexpr size_t kLayers = 4, kHeads = 16, kKvHeads = 4, kDim = 128, kPrompt = 300;
constexpr size_t kQDim = kHeads * kDim, kKvDim = kKvHeads * kDim, kQkv = kQDim + 2 * kKvDim;
constexpr size_t kSeq = kPrompt + 4;

struct Config {
    size_t num_layers, max_seq_len, num_kv_heads, head_dim;
};

int g_failures = 0;

void report(const char* name, bool ok, const char* detail = "") {
    std::printf("%s %s %s\n", ok ? "PASS" : "FAIL", name, detail);
    std::fflush(stdout);
    if (!ok) ++g_failures;
}

std::vector<__half> download(const __half* d, size_t n) {
    std::vector<__half> h(n);
    HIP_CHECK(hipMemcpy(h.data(), d, n * sizeof(__half), hipMemcpyDeviceToHost));
    return h;
}

bool same(const std::vector<__half>& a, const std::vector<__half>& b) {
    return a.size() == b.size() && std::memcmp(a.data(), b.data(), a.size() * 2) == 0;
}

// fp64 softmax(q . K^T / sqrt(D)) V over kv_len rows of one layer's cache
bool check_attention(const std::vector<__half>& q, const std::vector<__half>& k,
                     const std::vector<__half>& v, const std::vector<__half>& out,
                     size_t kv_len, double* maxd) {
    bool ok = true;
    *maxd = 0.0;
    const size_t group = kHeads / kKvHeads;
    std::vector<double> s(kv_len);
    for (size_t h = 0; h < kHeads; ++h) {
        const size_t g = h / group;
        double mx = -INFINITY;
        for (size_t t = 0; t < kv_len; ++t) {
            double acc = 0.0;
            for (size_t d = 0; d < kDim; ++d)
                acc += (double)__half2float(q[h * kDim + d]) *
                       __half2float(k[t * kKvDim + g * kDim + d]);
            s[t] = acc / std::sqrt((double)kDim);
            mx = std::max(mx, s[t]);
        }
        double den = 0.0;
        for (size_t t = 0; t < kv_len; ++t) den += (s[t] = std::exp(s[t] - mx));
        for (size_t d = 0; d < kDim; ++d) {
            double num = 0.0;
            for (size_t t = 0; t < kv_len; ++t)
                num += s[t] * __half2float(v[t * kKvDim + g * kDim + d]);
            const double e = num / den, a = __half2float(out[h * kDim + d]);
            const double diff = std::fabs(a - e);
            *maxd = std::max(*maxd, diff);
            if (!(diff <= 2e-3 + 1e-2 * std::fabs(e))) ok = false;
        }
    }
    return ok;
}

}  // namespace

int main() {
    const Config cfg{kLayers, kSeq, kKvHeads, kDim};
    KVCache graph_cache(cfg), eager_cache(cfg);
    RopeCache rope = create_rope_cache(kSeq, kDim, 5.0e6f);
    std::mt19937 gen(21);
    std::normal_distribution<float> nd;
    // per layer: the prompt's fused QKV rows, then one row per decode token
    std::vector<__half> h_prompt(kLayers * kPrompt * kQkv), h_tok(kLayers * 2 * kQkv);
    for (auto& x : h_prompt) x = __float2half(nd(gen));
    for (auto& x : h_tok) x = __float2half(nd(gen));
    __half *prompt, *tok_g, *tok_e, *out_p, *out_g, *out_e;
    HIP_CHECK(hipMalloc(&prompt, h_prompt.size() * 2));
    HIP_CHECK(hipMalloc(&tok_g, h_tok.size() * 2));
    HIP_CHECK(hipMalloc(&tok_e, h_tok.size() * 2));
    HIP_CHECK(hipMalloc(&out_p, kPrompt * kQDim * 2));
    HIP_CHECK(hipMalloc(&out_g, kLayers * kQDim * 2));
    HIP_CHECK(hipMalloc(&out_e, kLayers * kQDim * 2));
    HIP_CHECK(hipMemcpy(prompt, h_prompt.data(), h_prompt.size() * 2, hipMemcpyHostToDevice));
    HIP_CHECK(hipMemcpy(tok_g, h_tok.data(), h_tok.size() * 2, hipMemcpyHostToDevice));
    HIP_CHECK(hipMemcpy(tok_e, h_tok.data(), h_tok.size() * 2, hipMemcpyHostToDevice));
    const size_t cap = kHeads * ((kSeq + KV_CHUNK - 1) / KV_CHUNK);
    float *po, *pm, *ps, *po2, *pm2, *ps2;
    for (float** p : {&po, &po2}) HIP_CHECK(hipMalloc(p, cap * kDim * 4));
    for (float** p : {&pm, &ps, &pm2, &ps2}) HIP_CHECK(hipMalloc(p, cap * 4));

    // ---- prefill of the prompt into both caches (ModelInference::prefill)
    for (KVCache* c : {&graph_cache, &eager_cache}) {
        for (size_t l = 0; l < kLayers; ++l) {
            __half* q = prompt + l * kPrompt * kQkv;
            const bool apply = (l + 1) % 4 != 0;
            std::vector<__half> keep = download(q, kPrompt * kQkv);  // RoPE rotates in place
            launch_rope_and_store_kv(q, q + kQDim, q + kQDim + kKvDim, c->get_k_cache(l),
                                     c->get_v_cache(l), rope.d_cos, rope.d_sin, kPrompt, kHeads,
                                     kKvHeads, kDim, kQkv, kQkv, 0, apply);
            launch_causal_attention_prefill(q, c->get_k_cache(l), c->get_v_cache(l), out_p,
                                            kPrompt, kHeads, kKvHeads, kDim, kQkv, kKvDim);
            HIP_CHECK(hipGetLastError());
            HIP_CHECK(hipDeviceSynchronize());
            HIP_CHECK(hipMemcpy(q, keep.data(), keep.size() * 2, hipMemcpyHostToDevice));
        }
    }
    report("prefill_before_first_decode", true);

    // ---- first decode token: captured in global mode, the process's first
    // decode call (enqueue_decode, model_inference.hpp:361-387)
    hipStream_t stream;
    HIP_CHECK(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking));
    struct Nodes { hipGraphNode_t store_kv, attention, merge; };
    std::vector<Nodes> nodes(kLayers);
    auto enqueue = [&](KVCache& c, __half* tok, __half* out, size_t start_pos, hipStream_t s,
                       bool capture) {
        for (size_t l = 0; l < kLayers; ++l) {
            __half* q = tok + l * 2 * kQkv;
            const bool apply = (l + 1) % 4 != 0;
            launch_rope_and_store_kv(q, q + kQDim, q + kQDim + kKvDim, c.get_k_cache(l),
                                     c.get_v_cache(l), rope.d_cos, rope.d_sin, 1, kHeads,
                                     kKvHeads, kDim, kQkv, kQkv, start_pos, apply, s);
            if (capture) nodes[l].store_kv = last_captured_node(s);
            launch_causal_attention_decode_vectorized(
                q, c.get_k_cache(l), c.get_v_cache(l), out + l * kQDim, capture ? po : po2,
                capture ? pm : pm2, capture ? ps : ps2, 1, start_pos + 1, start_pos, kHeads,
                kKvHeads, kDim, kQkv, kKvDim, s, capture ? &nodes[l].attention : nullptr,
                capture ? &nodes[l].merge : nullptr);
        }
    };
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    HIP_CHECK(hipStreamBeginCapture(stream, hipStreamCaptureModeGlobal));
    enqueue(graph_cache, tok_g, out_g, kPrompt, stream, true);
    const hipError_t end = hipStreamEndCapture(stream, &graph);
    report("first_decode_inside_global_capture", end == hipSuccess, hipGetErrorString(end));
    if (end != hipSuccess) return g_failures;
    HIP_CHECK(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0));

    for (size_t t = 0; t < 2; ++t) {
        const size_t start_pos = kPrompt + t;
        if (t > 0) {
            // the next token's row of every layer, then patch (model_inference.hpp:105-123)
            for (size_t l = 0; l < kLayers; ++l) {
                HIP_CHECK(hipMemcpy(tok_g + l * 2 * kQkv, h_tok.data() + (l * 2 + 1) * kQkv,
                                    kQkv * 2, hipMemcpyHostToDevice));
                HIP_CHECK(hipMemcpy(tok_e + l * 2 * kQkv, h_tok.data() + (l * 2 + 1) * kQkv,
                                    kQkv * 2, hipMemcpyHostToDevice));
                const bool apply = (l + 1) % 4 != 0;
                update_rope_and_store_kv_node(exec, nodes[l].store_kv, start_pos, apply);
                update_causal_attention_decode_node(exec, nodes[l].attention, start_pos + 1);
                update_merge_attention_decode_node(exec, nodes[l].merge, start_pos + 1);
            }
        }
        HIP_CHECK(hipGraphLaunch(exec, stream));
        HIP_CHECK(hipStreamSynchronize(stream));
        enqueue(eager_cache, tok_e, out_e, start_pos, stream, false);
        HIP_CHECK(hipGetLastError());
        HIP_CHECK(hipStreamSynchronize(stream));
        bool bits = same(download(out_g, kLayers * kQDim), download(out_e, kLayers * kQDim)) &&
                    same(download(tok_g, kLayers * 2 * kQkv), download(tok_e, kLayers * 2 * kQkv));
        bool close = true;
        double worst = 0.0;
        for (size_t l = 0; l < kLayers; ++l) {
            const auto kg = download(graph_cache.get_k_cache(l), kSeq * kKvDim);
            const auto vg = download(graph_cache.get_v_cache(l), kSeq * kKvDim);
            bits = bits && same(kg, download(eager_cache.get_k_cache(l), kSeq * kKvDim)) &&
                   same(vg, download(eager_cache.get_v_cache(l), kSeq * kKvDim));
            double maxd = 0.0;
            close = check_attention(download(tok_g + l * 2 * kQkv, kQDim), kg, vg,
                                    download(out_g + l * kQDim, kQDim), start_pos + 1, &maxd) &&
                    close;
            worst = std::max(worst, maxd);
        }
        char detail[96];
        std::snprintf(detail, sizeof detail, "token %zu kv_len %zu max |diff| %.2e", t,
                      start_pos + 1, worst);
        report(t == 0 ? "captured_first_token_equals_eager" : "patched_token_equals_eager", bits,
               detail);
        report(t == 0 ? "captured_first_token_vs_fp64" : "patched_token_vs_fp64", close, detail);
    }
    HIP_CHECK(hipGraphExecDestroy(exec));
    HIP_CHECK(hipGraphDestroy(graph));
    HIP_CHECK(hipStreamDestroy(stream));
    return g_failures;
}
