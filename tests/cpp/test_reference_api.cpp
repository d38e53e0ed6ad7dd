// Exercises libattn_mi355x.so through the reference's own C++ interface
// (include/kernels/kernels.hpp, kv_cache.hpp, rope_cache.hpp, gpu_utils.hpp),
// the way the reference's tests and ModelInference use it:
//   1. Flash-Decode known-answer test, tests/test_causal_attention.cpp:152-228
//      (closed-form inputs, fp64 CPU softmax, output guards, 2e-3/2e-3).
//   2. RoPE + KV cache append, tests/test_rope.cpp:92-195 (interleaved/packed x
//      rotate/NoPE x start_pos {0, 2}; sentinel rows; other layer and sources
//      untouched; NoPE and V bit-exact), on seeded synthetic inputs.
//   3. Decode at every position vs the prefill row, test_causal_attention.cpp:80-150
//      (cache rows past L hold 123, output guards -123, interleaved Q stride).
//   4. A graph-captured decode step over several layers with per-step node
//      patching, model_inference.hpp:96-134, compared with eager launches.
//   5. launch_qkv_decode on the shapes, closed-form inputs, guards and
//      tolerance of tests/test_matrix_vec_mul.cpp:8-70 (beta = 0).
//   6. A graph-captured decode step built on the fused
//      launch_qkv_rope_and_store_kv_decode (patched per token) against eager
//      launch_qkv_decode + launch_rope_and_store_kv + decode, bit for bit.
//   7. A graph-captured decode step built on the fused
//      launch_rope_and_store_kv_decode (both nodes patched per token) against
//      eager launch_rope_and_store_kv + decode, bit for bit.
//   8. launch_qkv_gemm against an fp64 CPU product, and the fused
//      launch_qkv_gemm_rope_and_store_kv against the two launches, bit for bit.
//   9. launch_rope_and_store_kv_decode on a shape its fused kernels do not
//      serve (start_pos == kv_cache_len): with node handles it throws and
//      enqueues nothing; without, it equals the two reference launches.
// Prints one PASS/FAIL line per test; exit status is the number of failures.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <random>
#include <stdexcept>
#include <vector>

#include "../../include/gpu_utils.hpp"
#include "../../include/kernels/kernels.hpp"
#include "../../include/kv_cache.hpp"
#include "../../include/rope_cache.hpp"

namespace {

struct Config {
    size_t num_layers, max_seq_len, num_kv_heads, head_dim;
};

int g_failures = 0;

void report(const char* name, bool ok, const char* detail = "") {
    std::printf("%s %s %s\n", ok ? "PASS" : "FAIL", name, detail);
    std::fflush(stdout);
    if (!ok) ++g_failures;
}

template <typename T>
T* upload(const std::vector<T>& h) {
    T* d = nullptr;
    HIP_CHECK(hipMalloc(&d, h.size() * sizeof(T)));
    HIP_CHECK(hipMemcpy(d, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice));
    return d;
}

template <typename T>
std::vector<T> download(const T* d, size_t n) {
    std::vector<T> h(n);
    HIP_CHECK(hipMemcpy(h.data(), d, n * sizeof(T), hipMemcpyDeviceToHost));
    return h;
}

bool close(const __half* a, const __half* e, size_t n, float atol, float rtol, float* maxd) {
    bool ok = true;
    *maxd = 0.f;
    for (size_t i = 0; i < n; ++i) {
        const float x = __half2float(a[i]), y = __half2float(e[i]);
        const float d = std::fabs(x - y);
        *maxd = std::max(*maxd, d);
        if (!(d <= atol + rtol * std::fabs(y)) || !std::isfinite(x)) ok = false;
    }
    return ok;
}

bool same_bits(const __half* a, const __half* b, size_t n) {
    return std::memcmp(a, b, n * sizeof(__half)) == 0;
}

// ---------------------------------------------------------------- test 1
void test_flash_decode_kat() {
    const size_t lengths[] = {1, KV_CHUNK, KV_CHUNK + 1, 3 * KV_CHUNK + 1, 257};
    bool all = true;
    float worst = 0.f;
    for (size_t head_dim : {size_t(32), size_t(128)})
        for (size_t kv_heads : {size_t(1), size_t(2), size_t(4)})
            for (size_t len : lengths)
                for (bool padded : {false, true}) {
                    const size_t heads = 4, q_dim = heads * head_dim, kv_dim = kv_heads * head_dim;
                    const size_t stride = kv_dim + (padded ? 17 : 0);
                    std::vector<__half> q(q_dim), k((len + 2) * stride, __float2half(123.f));
                    auto v = k;
                    for (size_t i = 0; i < q.size(); ++i)
                        q[i] = __float2half(2.f * std::sin(float(i + 1) * .37f));
                    for (size_t t = 0; t < len; ++t)
                        for (size_t i = 0; i < kv_dim; ++i) {
                            k[t * stride + i] = __float2half(3.f * std::cos(float(t * kv_dim + i + 1) * .13f));
                            v[t * stride + i] = __float2half(std::sin(float(t * kv_dim + i + 3) * .19f));
                        }
                    std::vector<__half> expected(q_dim);
                    for (size_t hd = 0; hd < heads; ++hd) {
                        const size_t kh = hd / (heads / kv_heads);
                        std::vector<double> sc(len);
                        double mx = -INFINITY, den = 0.;
                        for (size_t t = 0; t < len; ++t) {
                            double dot = 0.;
                            for (size_t c = 0; c < head_dim; ++c)
                                dot += double(__half2float(q[hd * head_dim + c])) *
                                       __half2float(k[t * stride + kh * head_dim + c]);
                            sc[t] = dot / std::sqrt(double(head_dim));
                            mx = std::max(mx, sc[t]);
                        }
                        for (auto& x : sc) {
                            x = std::exp(x - mx);
                            den += x;
                        }
                        for (size_t c = 0; c < head_dim; ++c) {
                            double num = 0.;
                            for (size_t t = 0; t < len; ++t)
                                num += sc[t] * __half2float(v[t * stride + kh * head_dim + c]);
                            expected[hd * head_dim + c] = __float2half(float(num / den));
                        }
                    }
                    const size_t states = heads * ((len + KV_CHUNK - 1) / KV_CHUNK);
                    __half *dq = upload(q), *dk = upload(k), *dv = upload(v);
                    std::vector<__half> actual(q_dim + 2, __float2half(-123.f));
                    __half* out = upload(actual);
                    float *partial, *maximum, *sum;
                    HIP_CHECK(hipMalloc(&partial, states * head_dim * sizeof(float)));
                    HIP_CHECK(hipMalloc(&maximum, states * sizeof(float)));
                    HIP_CHECK(hipMalloc(&sum, states * sizeof(float)));
                    launch_causal_attention_decode(dq, dk, dv, out + 1, partial, maximum, sum, 1,
                                                   len, len - 1, heads, kv_heads, head_dim, 0,
                                                   padded ? stride : 0);
                    HIP_CHECK(hipGetLastError());
                    HIP_CHECK(hipDeviceSynchronize());
                    actual = download(out, q_dim + 2);
                    float md = 0.f;
                    const bool ok = close(actual.data() + 1, expected.data(), q_dim, 2e-3f, 2e-3f, &md) &&
                                    __half2float(actual.front()) == -123.f &&
                                    __half2float(actual.back()) == -123.f;
                    worst = std::max(worst, md);
                    if (!ok) {
                        std::printf("  KAT mismatch: D=%zu kv=%zu len=%zu padded=%d max|d|=%g\n",
                                    head_dim, kv_heads, len, (int)padded, md);
                        all = false;
                    }
                    for (void* p : {(void*)dq, (void*)dk, (void*)dv, (void*)out, (void*)partial,
                                    (void*)maximum, (void*)sum})
                        HIP_CHECK(hipFree(p));
                }
    char detail[64];
    std::snprintf(detail, sizeof detail, "(max |diff| %.2e)", worst);
    report("flash_decode_vs_cpu_softmax_kat", all, detail);
}

// CPU rotate-half with fp32 products rounded separately (rope.hip.cpp:53-57)
void cpu_rotate(__half* x, const __half* c, const __half* s, size_t half) {
    for (size_t i = 0; i < half; ++i) {
        const float x0 = __half2float(x[i]), x1 = __half2float(x[i + half]);
        const float cc = __half2float(c[i]), ss = __half2float(s[i]);
        volatile float p0 = x0 * cc, p1 = x1 * ss, p2 = x1 * cc, p3 = x0 * ss;
        x[i] = __float2half(p0 - p1);
        x[i + half] = __float2half(p2 + p3);
    }
}

// ---------------------------------------------------------------- test 2
void test_rope_and_store_kv() {
    const size_t heads = 16, kv_heads = 4, head_dim = 128, seq_len = 37;
    const size_t q_dim = heads * head_dim, kv_dim = kv_heads * head_dim;
    const size_t total_dim = q_dim + 2 * kv_dim;
    Config cfg{2, seq_len + 2, kv_heads, head_dim};
    KVCache cache(cfg);
    RopeCache rope = create_rope_cache(cfg.max_seq_len, head_dim, 5.0e6f);
    const auto cos_h = download(rope.d_cos, cfg.max_seq_len * head_dim / 2);
    const auto sin_h = download(rope.d_sin, cfg.max_seq_len * head_dim / 2);
    std::mt19937 gen(7);
    std::normal_distribution<float> nd;
    std::vector<__half> in_q(seq_len * q_dim), in_k(seq_len * kv_dim), in_v(seq_len * kv_dim);
    for (auto* vec : {&in_q, &in_k, &in_v})
        for (auto& x : *vec) x = __float2half(nd(gen));
    const size_t cache_elements = cfg.max_seq_len * kv_dim;
    const std::vector<__half> sentinel(cache_elements, __float2half(-123.f));
    bool all = true;
    for (bool interleaved : {false, true})
        for (bool rotate : {false, true})
            for (size_t start_pos : {size_t(0), size_t(2)}) {
                const size_t count = seq_len - start_pos;
                std::vector<__half> source;
                size_t q_off = 0, k_off, v_off, q_stride, kv_stride;
                if (interleaved) {
                    source.resize(count * total_dim);
                    k_off = q_dim;
                    v_off = q_dim + kv_dim;
                    q_stride = kv_stride = total_dim;
                    for (size_t t = 0; t < count; ++t) {
                        std::copy_n(in_q.data() + (start_pos + t) * q_dim, q_dim, source.data() + t * total_dim);
                        std::copy_n(in_k.data() + (start_pos + t) * kv_dim, kv_dim, source.data() + t * total_dim + k_off);
                        std::copy_n(in_v.data() + (start_pos + t) * kv_dim, kv_dim, source.data() + t * total_dim + v_off);
                    }
                } else {
                    source.insert(source.end(), in_q.begin() + start_pos * q_dim, in_q.end());
                    k_off = source.size();
                    source.insert(source.end(), in_k.begin() + start_pos * kv_dim, in_k.end());
                    v_off = source.size();
                    source.insert(source.end(), in_v.begin() + start_pos * kv_dim, in_v.end());
                    q_stride = q_dim;
                    kv_stride = kv_dim;
                }
                const auto original = source;
                __half* d_source = upload(source);
                for (size_t layer = 0; layer < cfg.num_layers; ++layer) {
                    HIP_CHECK(hipMemcpy(cache.get_k_cache(layer), sentinel.data(), cache_elements * 2, hipMemcpyHostToDevice));
                    HIP_CHECK(hipMemcpy(cache.get_v_cache(layer), sentinel.data(), cache_elements * 2, hipMemcpyHostToDevice));
                }
                launch_rope_and_store_kv(d_source + q_off, d_source + k_off, d_source + v_off,
                                         cache.get_k_cache(1), cache.get_v_cache(1), rope.d_cos,
                                         rope.d_sin, count, heads, kv_heads, head_dim, q_stride,
                                         kv_stride, start_pos, rotate);
                HIP_CHECK(hipGetLastError());
                HIP_CHECK(hipDeviceSynchronize());
                // expected K/V cache rows and Q
                auto exp_k = sentinel, exp_v = sentinel;
                std::vector<__half> exp_q(count * q_dim);
                for (size_t t = 0; t < count; ++t) {
                    const size_t pos = start_pos + t;
                    std::copy_n(in_k.data() + pos * kv_dim, kv_dim, exp_k.data() + pos * kv_dim);
                    std::copy_n(in_v.data() + pos * kv_dim, kv_dim, exp_v.data() + pos * kv_dim);
                    std::copy_n(in_q.data() + pos * q_dim, q_dim, exp_q.data() + t * q_dim);
                    if (rotate) {
                        for (size_t hd = 0; hd < kv_heads; ++hd)
                            cpu_rotate(exp_k.data() + pos * kv_dim + hd * head_dim,
                                       cos_h.data() + pos * head_dim / 2,
                                       sin_h.data() + pos * head_dim / 2, head_dim / 2);
                        for (size_t hd = 0; hd < heads; ++hd)
                            cpu_rotate(exp_q.data() + t * q_dim + hd * head_dim,
                                       cos_h.data() + pos * head_dim / 2,
                                       sin_h.data() + pos * head_dim / 2, head_dim / 2);
                    }
                }
                const auto act_k = download(cache.get_k_cache(1), cache_elements);
                const auto act_v = download(cache.get_v_cache(1), cache_elements);
                const auto act_src = download(d_source, source.size());
                bool ok = same_bits(act_k.data(), exp_k.data(), cache_elements) &&
                          same_bits(act_v.data(), exp_v.data(), cache_elements);
                for (const __half* p : {cache.get_k_cache(0), cache.get_v_cache(0)}) {
                    const auto untouched = download(p, cache_elements);
                    ok = ok && same_bits(untouched.data(), sentinel.data(), cache_elements);
                }
                for (size_t t = 0; t < count; ++t) {
                    ok = ok && same_bits(act_src.data() + q_off + t * q_stride, exp_q.data() + t * q_dim, q_dim);
                    ok = ok && same_bits(act_src.data() + k_off + t * kv_stride, original.data() + k_off + t * kv_stride, kv_dim);
                    ok = ok && same_bits(act_src.data() + v_off + t * kv_stride, original.data() + v_off + t * kv_stride, kv_dim);
                }
                if (!ok) {
                    std::printf("  rope mismatch: interleaved=%d rotate=%d start=%zu\n", (int)interleaved, (int)rotate, start_pos);
                    all = false;
                }
                HIP_CHECK(hipFree(d_source));
            }
    report("rope_and_store_kv_bitexact", all);
}

// ---------------------------------------------------------------- test 3
void test_decode_vs_prefill_rows() {
    const size_t heads = 16, kv_heads = 4, head_dim = 128, seq_len = 70;
    const size_t q_dim = heads * head_dim, kv_dim = kv_heads * head_dim;
    Config cfg{1, seq_len + 2, kv_heads, head_dim};
    KVCache cache(cfg);
    std::mt19937 gen(11);
    std::normal_distribution<float> nd;
    std::vector<__half> q(seq_len * q_dim);
    std::vector<__half> ck(cfg.max_seq_len * kv_dim, __float2half(123.f)), cv = ck;
    for (auto& x : q) x = __float2half(nd(gen));
    for (size_t i = 0; i < seq_len * kv_dim; ++i) {
        ck[i] = __float2half(nd(gen));
        cv[i] = __float2half(nd(gen));
    }
    HIP_CHECK(hipMemcpy(cache.get_k_cache(0), ck.data(), ck.size() * 2, hipMemcpyHostToDevice));
    HIP_CHECK(hipMemcpy(cache.get_v_cache(0), cv.data(), cv.size() * 2, hipMemcpyHostToDevice));
    __half* dq = upload(q);
    __half* dpre;
    HIP_CHECK(hipMalloc(&dpre, q.size() * 2));
    launch_causal_attention_prefill(dq, cache.get_k_cache(0), cache.get_v_cache(0), dpre, seq_len,
                                    heads, kv_heads, head_dim, q_dim, kv_dim);
    HIP_CHECK(hipGetLastError());
    HIP_CHECK(hipDeviceSynchronize());
    const auto pre = download(dpre, q.size());
    bool all = true;
    float worst = 0.f;
    for (bool interleaved : {false, true})
        for (size_t pos = 0; pos < seq_len; ++pos) {
            const size_t stride = interleaved ? q_dim + 2 * kv_dim : q_dim;
            std::vector<__half> input(stride, __float2half(-123.f));
            std::copy_n(q.data() + pos * q_dim, q_dim, input.data());
            __half* d_in = upload(input);
            std::vector<__half> output(3 * q_dim, __float2half(-123.f));
            const auto guards = output;
            __half* d_out = upload(output);
            const size_t states = heads * ((pos + 1 + KV_CHUNK - 1) / KV_CHUNK);
            float *po, *pm, *ps;
            HIP_CHECK(hipMalloc(&po, states * head_dim * 4));
            HIP_CHECK(hipMalloc(&pm, states * 4));
            HIP_CHECK(hipMalloc(&ps, states * 4));
            launch_causal_attention_decode_vectorized(d_in, cache.get_k_cache(0), cache.get_v_cache(0),
                                                      d_out + q_dim, po, pm, ps, 1, pos + 1, pos,
                                                      heads, kv_heads, head_dim,
                                                      interleaved ? stride : 0, 0);
            HIP_CHECK(hipGetLastError());
            HIP_CHECK(hipDeviceSynchronize());
            output = download(d_out, 3 * q_dim);
            float md = 0.f;
            const bool ok = close(output.data() + q_dim, pre.data() + pos * q_dim, q_dim, 4e-3f, 1e-2f, &md) &&
                            same_bits(output.data(), guards.data(), q_dim) &&
                            same_bits(output.data() + 2 * q_dim, guards.data(), q_dim);
            worst = std::max(worst, md);
            if (!ok) {
                std::printf("  decode/prefill mismatch at pos %zu interleaved %d (max %g)\n", pos, (int)interleaved, md);
                all = false;
            }
            for (void* p : {(void*)d_in, (void*)d_out, (void*)po, (void*)pm, (void*)ps}) HIP_CHECK(hipFree(p));
        }
    HIP_CHECK(hipFree(dq));
    HIP_CHECK(hipFree(dpre));
    char detail[64];
    std::snprintf(detail, sizeof detail, "(max |diff| %.2e)", worst);
    report("decode_vs_prefill_rows", all, detail);
}

// ---------------------------------------------------------------- test 4
// model_inference.hpp:96-134: capture the decode step once (per layer: RoPE +
// KV append, then Flash-Decode), then per token patch the three nodes of every
// layer and replay.  Each replay must equal eager launches of the same step.
void test_graph_decode_step() {
    const size_t layers = 4, heads = 16, kv_heads = 4, head_dim = 128;
    const size_t q_dim = heads * head_dim, kv_dim = kv_heads * head_dim, total = q_dim + 2 * kv_dim;
    const size_t prompt = 300, steps = 5;
    Config cfg{layers, prompt + steps + 1, kv_heads, head_dim};
    KVCache graph_cache(cfg), eager_cache(cfg);
    RopeCache rope = create_rope_cache(cfg.max_seq_len, head_dim, 5.0e6f);
    std::mt19937 gen(3);
    std::normal_distribution<float> nd;
    std::vector<__half> cache_init(cfg.num_layers * 2 * cfg.max_seq_len * kv_dim);
    for (auto& x : cache_init) x = __float2half(nd(gen));
    HIP_CHECK(hipMemcpy(graph_cache.get_k_cache(0), cache_init.data(), cache_init.size() * 2, hipMemcpyHostToDevice));
    HIP_CHECK(hipMemcpy(eager_cache.get_k_cache(0), cache_init.data(), cache_init.size() * 2, hipMemcpyHostToDevice));
    std::vector<std::vector<__half>> qkv_steps(steps, std::vector<__half>(layers * total));
    for (auto& st : qkv_steps)
        for (auto& x : st) x = __float2half(nd(gen));
    __half *d_qkv_g, *d_qkv_e, *d_out_g, *d_out_e;
    HIP_CHECK(hipMalloc(&d_qkv_g, layers * total * 2));
    HIP_CHECK(hipMalloc(&d_qkv_e, layers * total * 2));
    HIP_CHECK(hipMalloc(&d_out_g, layers * q_dim * 2));
    HIP_CHECK(hipMalloc(&d_out_e, layers * q_dim * 2));
    const size_t cap = heads * ((cfg.max_seq_len + KV_CHUNK - 1) / KV_CHUNK);
    float *po, *pm, *ps;
    HIP_CHECK(hipMalloc(&po, cap * head_dim * 4));
    HIP_CHECK(hipMalloc(&pm, cap * 4));
    HIP_CHECK(hipMalloc(&ps, cap * 4));
    hipStream_t stream;
    HIP_CHECK(hipStreamCreate(&stream));
    struct Nodes { hipGraphNode_t store_kv, attention, merge; };
    std::vector<Nodes> nodes(layers);
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    auto enqueue = [&](KVCache& cache, __half* qkv, __half* out, size_t start_pos, bool capture) {
        for (size_t l = 0; l < layers; ++l) {
            __half* a = qkv + l * total;
            const bool apply = (l + 1) % 4 != 0;
            launch_rope_and_store_kv(a, a + q_dim, a + q_dim + kv_dim, cache.get_k_cache(l),
                                     cache.get_v_cache(l), rope.d_cos, rope.d_sin, 1, heads,
                                     kv_heads, head_dim, total, total, start_pos, apply, stream);
            if (capture) nodes[l].store_kv = last_captured_node(stream);
            launch_causal_attention_decode_vectorized(
                a, cache.get_k_cache(l), cache.get_v_cache(l), out + l * q_dim, po, pm, ps, 1,
                start_pos + 1, start_pos, heads, kv_heads, head_dim, total, kv_dim, stream,
                capture ? &nodes[l].attention : nullptr, capture ? &nodes[l].merge : nullptr);
        }
    };
    bool all = true;
    for (size_t step = 0; step < steps; ++step) {
        const size_t start_pos = prompt + step;
        HIP_CHECK(hipMemcpy(d_qkv_g, qkv_steps[step].data(), layers * total * 2, hipMemcpyHostToDevice));
        HIP_CHECK(hipMemcpy(d_qkv_e, qkv_steps[step].data(), layers * total * 2, hipMemcpyHostToDevice));
        if (!exec) {
            HIP_CHECK(hipStreamBeginCapture(stream, hipStreamCaptureModeGlobal));
            enqueue(graph_cache, d_qkv_g, d_out_g, start_pos, true);
            HIP_CHECK(hipStreamEndCapture(stream, &graph));
            HIP_CHECK(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0));
        } else {
            for (size_t l = 0; l < layers; ++l) {
                update_rope_and_store_kv_node(exec, nodes[l].store_kv, start_pos, (l + 1) % 4 != 0);
                update_causal_attention_decode_node(exec, nodes[l].attention, start_pos + 1);
                update_merge_attention_decode_node(exec, nodes[l].merge, start_pos + 1);
            }
        }
        HIP_CHECK(hipGraphLaunch(exec, stream));
        HIP_CHECK(hipStreamSynchronize(stream));
        enqueue(eager_cache, d_qkv_e, d_out_e, start_pos, false);
        HIP_CHECK(hipStreamSynchronize(stream));
        const auto og = download(d_out_g, layers * q_dim), oe = download(d_out_e, layers * q_dim);
        const auto cg = download(graph_cache.get_k_cache(0), cache_init.size());
        const auto ce = download(eager_cache.get_k_cache(0), cache_init.size());
        const auto qg = download(d_qkv_g, layers * total), qe = download(d_qkv_e, layers * total);
        const bool ok = same_bits(og.data(), oe.data(), og.size()) &&
                        same_bits(cg.data(), ce.data(), cg.size()) &&
                        same_bits(qg.data(), qe.data(), qg.size());
        if (!ok) {
            std::printf("  graph/eager mismatch at step %zu\n", step);
            all = false;
        }
    }
    HIP_CHECK(hipGraphExecDestroy(exec));
    HIP_CHECK(hipGraphDestroy(graph));
    HIP_CHECK(hipStreamDestroy(stream));
    for (void* p : {(void*)d_qkv_g, (void*)d_qkv_e, (void*)d_out_g, (void*)d_out_e, (void*)po, (void*)pm, (void*)ps})
        HIP_CHECK(hipFree(p));
    report("graph_decode_step_node_patching", all);
}

// ---------------------------------------------------------------- test 5
void test_qkv_decode_reference_gemv() {
    struct Shape { size_t out_dim, in_dim, offset; };
    const Shape shapes[] = {{1, 1, 0},     {7, 31, 0},    {129, 129, 0}, {37, 2048, 0},
                            {19, 11008, 0}, {22016, 2048, 0}, {2048, 2048, 0}, {3072, 2048, 0},
                            {3, 0, 0},     {7, 8, 0},     {9, 2053, 0},  {5, 2056, 0},
                            {7, 4096, 0},  {5, 2056, 1}};
    hipStream_t stream;
    HIP_CHECK(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking));
    bool all = true;
    char detail[128] = "";
    for (const Shape& sh : shapes) {
        std::vector<__half> w(sh.out_dim * sh.in_dim + sh.offset + 1), x(sh.in_dim + sh.offset + 1);
        for (size_t i = 0; i < sh.out_dim * sh.in_dim; ++i)
            w[sh.offset + i] = __float2half((float)((int)(i % 29) - 14) / 64.0f);
        for (size_t i = 0; i < sh.in_dim; ++i)
            x[sh.offset + i] = __float2half((float)((int)(i % 17) - 8) / 16.0f);
        std::vector<__half> y(sh.out_dim + 2, __float2half(NAN));
        y.front() = y.back() = __float2half(123.0f);
        __half *dw = upload(w), *dx = upload(x), *dy = upload(y);
        launch_qkv_decode(dx + sh.offset, dy + 1, dw + sh.offset, sh.in_dim, sh.out_dim, stream);
        HIP_CHECK(hipGetLastError());
        HIP_CHECK(hipStreamSynchronize(stream));
        const auto got = download(dy, y.size());
        bool ok = __half2float(got.front()) == 123.0f && __half2float(got.back()) == 123.0f;
        for (size_t r = 0; r < sh.out_dim; ++r) {
            double e = 0.0;
            for (size_t c = 0; c < sh.in_dim; ++c)
                e += (double)__half2float(w[sh.offset + r * sh.in_dim + c]) *
                     __half2float(x[sh.offset + c]);
            const float a = __half2float(got[r + 1]);
            if (!std::isfinite(a) || std::fabs(a - e) > 1e-3 + 1e-3 * std::fabs(e)) ok = false;
        }
        if (!ok) {
            std::snprintf(detail, sizeof detail, "out=%zu in=%zu offset=%zu", sh.out_dim,
                          sh.in_dim, sh.offset);
            all = false;
        }
        for (void* p : {(void*)dw, (void*)dx, (void*)dy}) HIP_CHECK(hipFree(p));
    }
    // no rows: nothing launched, null pointers untouched
    launch_qkv_decode(nullptr, nullptr, nullptr, 2048, 0);
    HIP_CHECK(hipGetLastError());
    HIP_CHECK(hipStreamDestroy(stream));
    report("qkv_decode_reference_gemv_shapes", all, detail);
}

// ---------------------------------------------------------------- test 6
void test_graph_fused_qkv_decode_step() {
    const size_t layers = 4, heads = 16, kv_heads = 4, head_dim = 128, hidden = 2048;
    const size_t q_dim = heads * head_dim, kv_dim = kv_heads * head_dim, total = q_dim + 2 * kv_dim;
    const size_t prompt = 200, steps = 4;
    Config cfg{layers, prompt + steps + 1, kv_heads, head_dim};
    KVCache graph_cache(cfg), eager_cache(cfg);
    RopeCache rope = create_rope_cache(cfg.max_seq_len, head_dim, 5.0e6f);
    std::mt19937 gen(11);
    std::normal_distribution<float> nd;
    std::vector<__half> cache_init(cfg.num_layers * 2 * cfg.max_seq_len * kv_dim);
    for (auto& v : cache_init) v = __float2half(nd(gen));
    HIP_CHECK(hipMemcpy(graph_cache.get_k_cache(0), cache_init.data(), cache_init.size() * 2, hipMemcpyHostToDevice));
    HIP_CHECK(hipMemcpy(eager_cache.get_k_cache(0), cache_init.data(), cache_init.size() * 2, hipMemcpyHostToDevice));
    std::vector<__half> wts(layers * total * hidden);
    for (auto& v : wts) v = __float2half(nd(gen) / 45.0f);
    __half* d_w = upload(wts);
    std::vector<std::vector<__half>> x_steps(steps, std::vector<__half>(hidden));
    for (auto& st : x_steps)
        for (auto& v : st) v = __float2half(nd(gen));
    __half *d_x, *y_g, *y_e, *out_g, *out_e;
    HIP_CHECK(hipMalloc(&d_x, hidden * 2));
    HIP_CHECK(hipMalloc(&y_g, layers * total * 2));
    HIP_CHECK(hipMalloc(&y_e, layers * total * 2));
    HIP_CHECK(hipMalloc(&out_g, layers * q_dim * 2));
    HIP_CHECK(hipMalloc(&out_e, layers * q_dim * 2));
    const size_t cap = heads * ((cfg.max_seq_len + KV_CHUNK - 1) / KV_CHUNK);
    float *po, *pm, *ps;
    HIP_CHECK(hipMalloc(&po, cap * head_dim * 4));
    HIP_CHECK(hipMalloc(&pm, cap * 4));
    HIP_CHECK(hipMalloc(&ps, cap * 4));
    hipStream_t stream;
    HIP_CHECK(hipStreamCreate(&stream));
    struct Nodes { hipGraphNode_t store_kv, attention, merge; };
    std::vector<Nodes> nodes(layers);
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    // graph: the fused producer (model_inference.hpp:354-369 as one launch)
    auto enqueue_fused = [&](size_t start_pos) {
        for (size_t l = 0; l < layers; ++l) {
            __half* a = y_g + l * total;
            launch_qkv_rope_and_store_kv_decode(d_x, a, d_w + l * total * hidden,
                                                graph_cache.get_k_cache(l),
                                                graph_cache.get_v_cache(l), rope.d_cos,
                                                rope.d_sin, hidden, heads, kv_heads, head_dim,
                                                start_pos, (l + 1) % 4 != 0, stream);
            nodes[l].store_kv = last_captured_node(stream);
            launch_causal_attention_decode_vectorized(
                a, graph_cache.get_k_cache(l), graph_cache.get_v_cache(l), out_g + l * q_dim, po,
                pm, ps, 1, start_pos + 1, start_pos, heads, kv_heads, head_dim, total, kv_dim,
                stream, &nodes[l].attention, &nodes[l].merge);
        }
    };
    // eager: the reference's two launches
    auto enqueue_two = [&](size_t start_pos) {
        for (size_t l = 0; l < layers; ++l) {
            __half* a = y_e + l * total;
            launch_qkv_decode(d_x, a, d_w + l * total * hidden, hidden, total, stream);
            launch_rope_and_store_kv(a, a + q_dim, a + q_dim + kv_dim, eager_cache.get_k_cache(l),
                                     eager_cache.get_v_cache(l), rope.d_cos, rope.d_sin, 1,
                                     heads, kv_heads, head_dim, total, total, start_pos,
                                     (l + 1) % 4 != 0, stream);
            launch_causal_attention_decode_vectorized(
                a, eager_cache.get_k_cache(l), eager_cache.get_v_cache(l), out_e + l * q_dim, po,
                pm, ps, 1, start_pos + 1, start_pos, heads, kv_heads, head_dim, total, kv_dim,
                stream, nullptr, nullptr);
        }
    };
    bool all = true;
    for (size_t step = 0; step < steps; ++step) {
        const size_t start_pos = prompt + step;
        HIP_CHECK(hipMemcpy(d_x, x_steps[step].data(), hidden * 2, hipMemcpyHostToDevice));
        if (!exec) {
            HIP_CHECK(hipStreamBeginCapture(stream, hipStreamCaptureModeGlobal));
            enqueue_fused(start_pos);
            HIP_CHECK(hipStreamEndCapture(stream, &graph));
            HIP_CHECK(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0));
        } else {
            for (size_t l = 0; l < layers; ++l) {
                update_qkv_rope_and_store_kv_node(exec, nodes[l].store_kv, start_pos,
                                                  (l + 1) % 4 != 0);
                update_causal_attention_decode_node(exec, nodes[l].attention, start_pos + 1);
                update_merge_attention_decode_node(exec, nodes[l].merge, start_pos + 1);
            }
        }
        HIP_CHECK(hipGraphLaunch(exec, stream));
        HIP_CHECK(hipStreamSynchronize(stream));
        enqueue_two(start_pos);
        HIP_CHECK(hipStreamSynchronize(stream));
        const auto og = download(out_g, layers * q_dim), oe = download(out_e, layers * q_dim);
        const auto yg = download(y_g, layers * total), ye = download(y_e, layers * total);
        const auto cg = download(graph_cache.get_k_cache(0), cache_init.size());
        const auto ce = download(eager_cache.get_k_cache(0), cache_init.size());
        if (!(same_bits(og.data(), oe.data(), og.size()) && same_bits(yg.data(), ye.data(), yg.size()) &&
              same_bits(cg.data(), ce.data(), cg.size()))) {
            std::printf("  fused graph / two-launch mismatch at step %zu\n", step);
            all = false;
        }
    }
    HIP_CHECK(hipGraphExecDestroy(exec));
    HIP_CHECK(hipGraphDestroy(graph));
    HIP_CHECK(hipStreamDestroy(stream));
    for (void* p : {(void*)d_w, (void*)d_x, (void*)y_g, (void*)y_e, (void*)out_g, (void*)out_e,
                    (void*)po, (void*)pm, (void*)ps})
        HIP_CHECK(hipFree(p));
    report("graph_fused_qkv_decode_step", all);
}

// ---------------------------------------------------------------- test 7
// launch_rope_and_store_kv_decode (not in the reference) captured per layer
// and patched per step with update_rope_and_store_kv_decode_nodes: q, the
// caches and the outputs equal the reference's launch_rope_and_store_kv +
// launch_causal_attention_decode_vectorized bit for bit at every step.
void test_graph_fused_rope_decode_step() {
    const size_t layers = 4, heads = 16, kv_heads = 4, head_dim = 128;
    const size_t q_dim = heads * head_dim, kv_dim = kv_heads * head_dim, total = q_dim + 2 * kv_dim;
    const size_t prompt = 3000, steps = 4;
    Config cfg{layers, prompt + steps + 1, kv_heads, head_dim};
    KVCache graph_cache(cfg), eager_cache(cfg);
    RopeCache rope = create_rope_cache(cfg.max_seq_len, head_dim, 5.0e6f);
    std::mt19937 gen(12);
    std::normal_distribution<float> nd;
    std::vector<__half> cache_init(cfg.num_layers * 2 * cfg.max_seq_len * kv_dim);
    for (auto& v : cache_init) v = __float2half(nd(gen));
    HIP_CHECK(hipMemcpy(graph_cache.get_k_cache(0), cache_init.data(), cache_init.size() * 2, hipMemcpyHostToDevice));
    HIP_CHECK(hipMemcpy(eager_cache.get_k_cache(0), cache_init.data(), cache_init.size() * 2, hipMemcpyHostToDevice));
    __half *y_g, *y_e, *out_g, *out_e;
    HIP_CHECK(hipMalloc(&y_g, layers * total * 2));
    HIP_CHECK(hipMalloc(&y_e, layers * total * 2));
    HIP_CHECK(hipMalloc(&out_g, layers * q_dim * 2));
    HIP_CHECK(hipMalloc(&out_e, layers * q_dim * 2));
    const size_t cap = heads * ((cfg.max_seq_len + KV_CHUNK - 1) / KV_CHUNK);
    float *po, *pm, *ps;
    HIP_CHECK(hipMalloc(&po, cap * head_dim * 4));
    HIP_CHECK(hipMalloc(&pm, cap * 4));
    HIP_CHECK(hipMalloc(&ps, cap * 4));
    hipStream_t stream;
    HIP_CHECK(hipStreamCreate(&stream));
    struct Nodes { hipGraphNode_t attention, merge; };
    std::vector<Nodes> nodes(layers);
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    auto enqueue_fused = [&](size_t start_pos) {
        for (size_t l = 0; l < layers; ++l) {
            __half* a = y_g + l * total;
            launch_rope_and_store_kv_decode(a, a + q_dim, a + q_dim + kv_dim,
                                            graph_cache.get_k_cache(l), graph_cache.get_v_cache(l),
                                            rope.d_cos, rope.d_sin, out_g + l * q_dim, po, pm, ps,
                                            start_pos + 1, start_pos, heads, kv_heads, head_dim,
                                            (l + 1) % 4 != 0, stream, &nodes[l].attention,
                                            &nodes[l].merge);
        }
    };
    auto enqueue_two = [&](size_t start_pos) {
        for (size_t l = 0; l < layers; ++l) {
            __half* a = y_e + l * total;
            launch_rope_and_store_kv(a, a + q_dim, a + q_dim + kv_dim, eager_cache.get_k_cache(l),
                                     eager_cache.get_v_cache(l), rope.d_cos, rope.d_sin, 1,
                                     heads, kv_heads, head_dim, total, total, start_pos,
                                     (l + 1) % 4 != 0, stream);
            launch_causal_attention_decode_vectorized(
                a, eager_cache.get_k_cache(l), eager_cache.get_v_cache(l), out_e + l * q_dim, po,
                pm, ps, 1, start_pos + 1, start_pos, heads, kv_heads, head_dim, total, kv_dim,
                stream, nullptr, nullptr);
        }
    };
    bool all = true;
    std::vector<__half> qkv(layers * total);
    for (size_t step = 0; step < steps; ++step) {
        const size_t start_pos = prompt + step;
        for (auto& v : qkv) v = __float2half(nd(gen));
        HIP_CHECK(hipMemcpy(y_g, qkv.data(), qkv.size() * 2, hipMemcpyHostToDevice));
        HIP_CHECK(hipMemcpy(y_e, qkv.data(), qkv.size() * 2, hipMemcpyHostToDevice));
        if (!exec) {
            HIP_CHECK(hipStreamBeginCapture(stream, hipStreamCaptureModeGlobal));
            enqueue_fused(start_pos);
            HIP_CHECK(hipStreamEndCapture(stream, &graph));
            HIP_CHECK(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0));
        } else {
            for (size_t l = 0; l < layers; ++l)
                update_rope_and_store_kv_decode_nodes(exec, nodes[l].attention, nodes[l].merge,
                                                      start_pos + 1, start_pos, (l + 1) % 4 != 0);
        }
        HIP_CHECK(hipGraphLaunch(exec, stream));
        HIP_CHECK(hipStreamSynchronize(stream));
        enqueue_two(start_pos);
        HIP_CHECK(hipStreamSynchronize(stream));
        const auto og = download(out_g, layers * q_dim), oe = download(out_e, layers * q_dim);
        const auto yg = download(y_g, layers * total), ye = download(y_e, layers * total);
        const auto cg = download(graph_cache.get_k_cache(0), cache_init.size());
        const auto ce = download(eager_cache.get_k_cache(0), cache_init.size());
        if (!(same_bits(og.data(), oe.data(), og.size()) && same_bits(yg.data(), ye.data(), yg.size()) &&
              same_bits(cg.data(), ce.data(), cg.size()))) {
            std::printf("  fused rope+decode graph / two-launch mismatch at step %zu\n", step);
            all = false;
        }
    }
    HIP_CHECK(hipGraphExecDestroy(exec));
    HIP_CHECK(hipGraphDestroy(graph));
    HIP_CHECK(hipStreamDestroy(stream));
    for (void* p : {(void*)y_g, (void*)y_e, (void*)out_g, (void*)out_e, (void*)po, (void*)pm,
                    (void*)ps})
        HIP_CHECK(hipFree(p));
    report("graph_fused_rope_decode_step", all);
}

// ---------------------------------------------------------------- test 8
void test_qkv_gemm_prefill() {
    const size_t heads = 16, kv_heads = 4, head_dim = 128, hidden = 2048, tokens = 70;
    const size_t q_dim = heads * head_dim, kv_dim = kv_heads * head_dim, total = q_dim + 2 * kv_dim;
    Config cfg{2, tokens + 8, kv_heads, head_dim};
    KVCache fused_cache(cfg), two_cache(cfg);
    const size_t cache_bytes = cfg.num_layers * 2 * cfg.max_seq_len * kv_dim * 2;
    HIP_CHECK(hipMemset(fused_cache.get_k_cache(0), 0, cache_bytes));
    HIP_CHECK(hipMemset(two_cache.get_k_cache(0), 0, cache_bytes));
    RopeCache rope = create_rope_cache(cfg.max_seq_len, head_dim, 5.0e6f);
    std::mt19937 gen(21);
    std::normal_distribution<float> nd;
    std::vector<__half> x(tokens * hidden), w(total * hidden);
    for (auto& v : x) v = __float2half(nd(gen));
    for (auto& v : w) v = __float2half(nd(gen) / 45.0f);
    __half *dx = upload(x), *dw = upload(w), *y1, *y2;
    HIP_CHECK(hipMalloc(&y1, tokens * total * 2));
    HIP_CHECK(hipMalloc(&y2, tokens * total * 2));
    // the GEMM against an fp64 CPU product (null stream, as the reference)
    launch_qkv_gemm(dx, y1, dw, tokens, hidden, total);
    HIP_CHECK(hipDeviceSynchronize());
    const auto got = download(y1, tokens * total);
    std::vector<double> wd(w.size());
    for (size_t i = 0; i < w.size(); ++i) wd[i] = __half2float(w[i]);
    bool gemm_ok = true;
    for (size_t m = 0; m < tokens; ++m)
        for (size_t r = 0; r < total; ++r) {
            double e = 0.0;
            for (size_t c = 0; c < hidden; ++c) e += wd[r * hidden + c] * __half2float(x[m * hidden + c]);
            const float a = __half2float(got[m * total + r]);
            if (!std::isfinite(a) || std::fabs(a - e) > 2e-3 + 1e-2 * std::fabs(e)) gemm_ok = false;
        }
    report("qkv_gemm_vs_fp64", gemm_ok);
    // fused projection + RoPE + append against the two launches, layer 1 with
    // rotation at start_pos 5, layer 0 NoPE at 0
    bool fused_ok = true;
    for (size_t l = 0; l < 2; ++l) {
        const size_t start = l == 1 ? 5 : 0;
        const bool apply = l == 1;
        launch_qkv_gemm_rope_and_store_kv(dx, y1, dw, fused_cache.get_k_cache(l),
                                          fused_cache.get_v_cache(l), rope.d_cos, rope.d_sin,
                                          tokens, hidden, heads, kv_heads, head_dim, start, apply);
        launch_qkv_gemm(dx, y2, dw, tokens, hidden, total);
        launch_rope_and_store_kv(y2, y2 + q_dim, y2 + q_dim + kv_dim, two_cache.get_k_cache(l),
                                 two_cache.get_v_cache(l), rope.d_cos, rope.d_sin, tokens, heads,
                                 kv_heads, head_dim, total, total, start, apply);
        HIP_CHECK(hipDeviceSynchronize());
        const auto a = download(y1, tokens * total), b = download(y2, tokens * total);
        const auto ca = download(fused_cache.get_k_cache(l), 2 * cfg.max_seq_len * kv_dim);
        const auto cb = download(two_cache.get_k_cache(l), 2 * cfg.max_seq_len * kv_dim);
        if (!same_bits(a.data(), b.data(), a.size()) || !same_bits(ca.data(), cb.data(), ca.size()))
            fused_ok = false;
    }
    report("qkv_gemm_fused_rope_store_kv_bitexact", fused_ok);
    for (void* p : {(void*)dx, (void*)dw, (void*)y1, (void*)y2}) HIP_CHECK(hipFree(p));
}

// ---------------------------------------------------------------- test 9
void test_fused_rope_decode_other_shape() {
    const size_t heads = 8, kv_heads = 2, head_dim = 128, L = 40, start_pos = L;
    const size_t q_dim = heads * head_dim, kv_dim = kv_heads * head_dim;
    Config cfg{1, L + 4, kv_heads, head_dim};
    KVCache fused_cache(cfg), two_cache(cfg);
    RopeCache rope = create_rope_cache(cfg.max_seq_len, head_dim, 5.0e6f);
    std::mt19937 gen(9);
    std::normal_distribution<float> nd;
    std::vector<__half> cache_init(2 * cfg.max_seq_len * kv_dim), qkv(q_dim + 2 * kv_dim);
    for (auto& v : cache_init) v = __float2half(nd(gen));
    for (auto& v : qkv) v = __float2half(nd(gen));
    for (KVCache* c : {&fused_cache, &two_cache})
        HIP_CHECK(hipMemcpy(c->get_k_cache(0), cache_init.data(), cache_init.size() * 2,
                            hipMemcpyHostToDevice));
    __half* a_f = upload(qkv);
    __half* a_t = upload(qkv);
    __half *out_f, *out_t;
    HIP_CHECK(hipMalloc(&out_f, q_dim * 2));
    HIP_CHECK(hipMalloc(&out_t, q_dim * 2));
    HIP_CHECK(hipMemset(out_f, 0, q_dim * 2));
    HIP_CHECK(hipMemset(out_t, 0, q_dim * 2));
    const size_t cap = heads * ((cfg.max_seq_len + KV_CHUNK - 1) / KV_CHUNK);
    float *po, *pm, *ps;
    HIP_CHECK(hipMalloc(&po, cap * head_dim * 4));
    HIP_CHECK(hipMalloc(&pm, cap * 4));
    HIP_CHECK(hipMalloc(&ps, cap * 4));
    auto fused = [&](hipGraphNode_t* an, hipGraphNode_t* mn) {
        launch_rope_and_store_kv_decode(a_f, a_f + q_dim, a_f + q_dim + kv_dim,
                                        fused_cache.get_k_cache(0), fused_cache.get_v_cache(0),
                                        rope.d_cos, rope.d_sin, out_f, po, pm, ps, L, start_pos,
                                        heads, kv_heads, head_dim, true, nullptr, an, mn);
    };
    hipGraphNode_t an = nullptr, mn = nullptr;
    bool threw = false;
    try {
        fused(&an, &mn);
    } catch (const std::runtime_error&) {
        threw = true;
    }
    HIP_CHECK(hipDeviceSynchronize());
    bool untouched = same_bits(download(out_f, q_dim).data(), download(out_t, q_dim).data(),
                               q_dim) &&
                     same_bits(download(fused_cache.get_k_cache(0), cache_init.size()).data(),
                               cache_init.data(), cache_init.size());
    bool eager_ok = true;
    try {
        fused(nullptr, nullptr);
    } catch (const std::runtime_error&) {
        eager_ok = false;
    }
    launch_rope_and_store_kv(a_t, a_t + q_dim, a_t + q_dim + kv_dim, two_cache.get_k_cache(0),
                             two_cache.get_v_cache(0), rope.d_cos, rope.d_sin, 1, heads, kv_heads,
                             head_dim, 0, 0, start_pos, true, nullptr);
    launch_causal_attention_decode(a_t, two_cache.get_k_cache(0), two_cache.get_v_cache(0), out_t,
                                   po, pm, ps, 1, L, start_pos, heads, kv_heads, head_dim, 0, 0);
    HIP_CHECK(hipDeviceSynchronize());
    const bool same =
        same_bits(download(out_f, q_dim).data(), download(out_t, q_dim).data(), q_dim) &&
        same_bits(download(a_f, qkv.size()).data(), download(a_t, qkv.size()).data(),
                  qkv.size()) &&
        same_bits(download(fused_cache.get_k_cache(0), cache_init.size()).data(),
                  download(two_cache.get_k_cache(0), cache_init.size()).data(),
                  cache_init.size());
    char detail[96];
    std::snprintf(detail, sizeof detail, "threw=%d untouched=%d eager=%d same=%d", threw,
                  untouched, eager_ok, same);
    for (void* p : {(void*)a_f, (void*)a_t, (void*)out_f, (void*)out_t, (void*)po, (void*)pm,
                    (void*)ps})
        HIP_CHECK(hipFree(p));
    report("fused_rope_decode_other_shape_throws_or_falls_back",
           threw && untouched && eager_ok && same, detail);
}

}  // namespace

int main() {
    int dev = 0;
    HIP_CHECK(hipSetDevice(dev));
    test_flash_decode_kat();
    test_rope_and_store_kv();
    test_decode_vs_prefill_rows();
    test_graph_decode_step();
    test_qkv_decode_reference_gemv();
    test_graph_fused_qkv_decode_step();
    test_graph_fused_rope_decode_step();
    test_qkv_gemm_prefill();
    test_fused_rope_decode_other_shape();
    std::printf("%d failure(s)\n", g_failures);
    return g_failures;
}
