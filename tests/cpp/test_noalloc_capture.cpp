// attn_decode_noalloc whose FIRST call in the process is made inside a
// hipStreamCaptureModeGlobal capture (the use it exists for: code under graph
// capture that must not allocate).  That first call also looks up the device
// address of the library's array.  Either the lookup works under capture
// (the call is captured, the graph is launched and must equal an eager
// attn_decode_noalloc call and attn_decode with a workspace bit for bit), or
// it is refused (the call returns the error, the capture is ended, and the
// next call, eager, must look the address up again, succeed and equal
// attn_decode bit for bit: a failed lookup is not kept).  Run as its own
// process; prints PASS/FAIL lines and exits with the number of failures.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <random>
#include <vector>

#include "../../include/attn_mi355x.h"

namespace {

constexpr size_t kHeads = 16, kKvHeads = 4, kDim = 128, kLen = 4096;
constexpr size_t kQDim = kHeads * kDim, kKvDim = kKvHeads * kDim;

int g_failures = 0;

void report(const char* name, bool ok, const char* detail = "") {
    std::printf("%s %s %s\n", ok ? "PASS" : "FAIL", name, detail);
    std::fflush(stdout);
    if (!ok) ++g_failures;
}

#define CHECK(x)                                                                        \
    do {                                                                                \
        const hipError_t e_ = (x);                                                      \
        if (e_ != hipSuccess) {                                                         \
            std::printf("FAIL %s: %s\n", #x, hipGetErrorString(e_));                     \
            return 1;                                                                   \
        }                                                                               \
    } while (0)

std::vector<uint16_t> random_f16(size_t n, uint32_t seed) {
    std::mt19937 rng(seed);
    std::normal_distribution<float> d(0.f, 1.f);
    std::vector<uint16_t> h(n);
    for (auto& x : h) {
        const _Float16 v = (_Float16)d(rng);
        std::memcpy(&x, &v, 2);
    }
    return h;
}

}  // namespace

int main() {
    const auto hq = random_f16(kQDim, 11), hk = random_f16(kLen * kKvDim, 12),
               hv = random_f16(kLen * kKvDim, 13);
    attn_f16_t *q, *k, *v, *out_a, *out_b, *out_ref;
    CHECK(hipMalloc(&q, kQDim * 2));
    CHECK(hipMalloc(&k, kLen * kKvDim * 2));
    CHECK(hipMalloc(&v, kLen * kKvDim * 2));
    CHECK(hipMalloc(&out_a, kQDim * 2));
    CHECK(hipMalloc(&out_b, kQDim * 2));
    CHECK(hipMalloc(&out_ref, kQDim * 2));
    CHECK(hipMemcpy(q, hq.data(), kQDim * 2, hipMemcpyHostToDevice));
    CHECK(hipMemcpy(k, hk.data(), kLen * kKvDim * 2, hipMemcpyHostToDevice));
    CHECK(hipMemcpy(v, hv.data(), kLen * kKvDim * 2, hipMemcpyHostToDevice));
    CHECK(hipMemset(out_a, 0xff, kQDim * 2));
    CHECK(hipMemset(out_b, 0xff, kQDim * 2));
    const size_t states = attn_decode_workspace_states(kHeads, kLen);
    float *po, *pm, *ps;
    CHECK(hipMalloc(&po, states * kDim * 4));
    CHECK(hipMalloc(&pm, states * 4));
    CHECK(hipMalloc(&ps, states * 4));
    hipStream_t stream;
    CHECK(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking));
    CHECK(hipDeviceSynchronize());

    // the process's first attn_decode_noalloc call, under global capture
    CHECK(hipStreamBeginCapture(stream, hipStreamCaptureModeGlobal));
    const int rc = attn_decode_noalloc(q, k, v, out_a, kLen, kHeads, kKvHeads, kDim, 0, stream);
    hipGraph_t graph = nullptr;
    const hipError_t end = hipStreamEndCapture(stream, &graph);
    (void)hipGetLastError();
    char detail[160];
    std::snprintf(detail, sizeof detail, "(first call under global capture: rc %d, end capture %d)",
                  rc, (int)end);
    const bool captured = rc == 0 && end == hipSuccess && graph != nullptr;
    if (captured) {
        hipGraphExec_t exec;
        CHECK(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0));
        CHECK(hipGraphLaunch(exec, stream));
        CHECK(hipStreamSynchronize(stream));
        CHECK(hipGraphExecDestroy(exec));
        report("first_noalloc_call_captured", true, detail);
    } else {
        // refused under capture: reported, and nothing was enqueued
        report("first_noalloc_call_refused_under_capture", rc != 0, detail);
    }
    if (graph) CHECK(hipGraphDestroy(graph));

    // an eager call after it: the address is looked up again if it was not kept
    const int rc2 = attn_decode_noalloc(q, k, v, out_b, kLen, kHeads, kKvHeads, kDim, 0, stream);
    CHECK(hipStreamSynchronize(stream));
    report("eager_noalloc_call_after_capture", rc2 == 0);
    const int rc3 = attn_decode(q, k, v, out_ref, po, pm, ps, 1, kLen, kLen - 1, kHeads, kKvHeads,
                                kDim, 0, 0, stream, nullptr, nullptr);
    CHECK(hipStreamSynchronize(stream));
    report("workspace_decode", rc3 == 0);
    std::vector<uint16_t> a(kQDim), b(kQDim), r(kQDim);
    CHECK(hipMemcpy(a.data(), out_a, kQDim * 2, hipMemcpyDeviceToHost));
    CHECK(hipMemcpy(b.data(), out_b, kQDim * 2, hipMemcpyDeviceToHost));
    CHECK(hipMemcpy(r.data(), out_ref, kQDim * 2, hipMemcpyDeviceToHost));
    report("eager_noalloc_equals_workspace_decode", b == r);
    if (captured) report("captured_noalloc_equals_workspace_decode", a == r);
    return g_failures;
}
