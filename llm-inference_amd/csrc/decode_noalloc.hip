// attn_decode_noalloc: Flash-Decode without a caller workspace, for callers
// that cannot allocate device memory (code under graph capture that must not
// call hipMalloc, tight serving loops, harnesses that forbid it).  It runs the
// same plan and kernels as attn_decode (split kernel, merge kernel; the split
// kernel alone for the short contexts decoded by one workgroup per KV head); the
// partial states (D fp16 outputs and two floats per query head and split) live in a
// file-scope device array instead of the caller's partial_out/max/sum.
//
// The array is per GPU and lives until the process ends.  Its device address
// is taken with hipGetSymbolAddress (the array's name is only a host-side
// stand-in) on the first call on that device, with that device current, and
// kept once that lookup has succeeded; kernels receive addresses inside it as
// their partial state pointers.  Every call on one GPU shares the array and leaves its
// states there; the split kernel writes every state the merge kernel reads
// before the merge runs, so nothing needs to start at zero.  Calls that
// overlap on one GPU (different streams without ordering) race on the array
// and must not be issued.  Nothing here calls hipMalloc, hipFree or an
// allocating library routine.
#include "attn_internal.hpp"
#include "../../include/attn_mi355x.h"

#include <atomic>
#include <mutex>

namespace attn {
namespace {

constexpr size_t kScratchBytes = ATTN_DECODE_NOALLOC_SCRATCH_BYTES;
// bytes of one (query head, split) partial state: D fp16 outputs, fp32 max and sum
constexpr size_t kStateBytes = 128 * 2 + 2 * 4;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
// per device: the array's address once hipGetSymbolAddress has returned it
std::atomic<void*> g_scratch[kMaxDevices];
std::mutex g_scratch_mu;

// The device address of `scratch` on `device` (the current device).  Only a
// successful lookup is kept: a call that fails (for example one made while a
// global-mode stream capture forbids it) returns the error and the next call
// on that device asks again.
hipError_t scratch_on(int device, void** ptr) {
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    void* p = g_scratch[device].load(std::memory_order_acquire);
    if (!p) {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        p = g_scratch[device].load(std::memory_order_relaxed);
        if (!p) {
            const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
            if (e != hipSuccess) return e;
            if (!p) return hipErrorInvalidSymbol;
            g_scratch[device].store(p, std::memory_order_release);
        }
    }
    *ptr = p;
    return hipSuccess;
}

}  // namespace
}  // namespace attn

using namespace attn;

extern "C" int attn_decode_noalloc(const attn_f16_t* q, const attn_f16_t* k_cache,
                                   const attn_f16_t* v_cache, attn_f16_t* out, size_t kv_len,
                                   size_t num_heads, size_t num_kv_heads, size_t head_dim,
                                   size_t kv_stride, hipStream_t stream) {
    // the no-op shapes of attn_decode (causal_attention.hip.cpp:860-866, :945-946)
    if (kv_len == 0 || num_kv_heads == 0 || head_dim == 0) return 0;
    if (num_heads % num_kv_heads != 0) return 0;
    if (kv_len > 0xffffffffull || num_heads > 0xffffffffull || head_dim > 0xffffffffull)
        return (int)hipErrorInvalidValue;
    if (!q || !k_cache || !v_cache || !out) return (int)hipErrorInvalidValue;
    const size_t kvs = kv_stride ? kv_stride : num_kv_heads * head_dim;
    int device = 0;
    hipError_t e = hipGetDevice(&device);
    if (e != hipSuccess) return (int)e;
    const DecodePlan p = plan_decode((uint32_t)kv_len, (uint32_t)num_heads,
                                     (uint32_t)num_kv_heads, (uint32_t)head_dim, kvs, q,
                                     k_cache, v_cache, device, true);
    if (p.path == 0) {
        // shapes off the MFMA path take attn_decode's generic kernel, which
        // has no partial states
        return attn_decode(q, k_cache, v_cache, out, nullptr, nullptr, nullptr, 1, kv_len,
                           kv_len - 1, num_heads, num_kv_heads, head_dim, 0, kv_stride, stream,
                           nullptr, nullptr);
    }
    // the states of this plan must fit the array
    const size_t states = (size_t)num_heads * p.nstate;
    if (states * kStateBytes > kScratchBytes) return (int)hipErrorInvalidValue;
    void* ws = nullptr;
    e = scratch_on(device, &ws);
    if (e != hipSuccess) return (int)e;
    DecodeArgs a{};
    a.q = reinterpret_cast<const f16*>(q);
    a.k = reinterpret_cast<const f16*>(k_cache);
    a.v = reinterpret_cast<const f16*>(v_cache);
    a.out = reinterpret_cast<f16*>(out);
    a.part_out = static_cast<float*>(ws);
    a.part_max = a.part_out + states * 64;  // after states x 128 fp16 outputs
    a.part_sum = a.part_max + states;
    a.kv_stride = kvs;
    a.kv_len = (uint32_t)kv_len;
    a.num_heads = (uint32_t)num_heads;
    a.num_kv_heads = (uint32_t)num_kv_heads;
    a.group = (uint32_t)(num_heads / num_kv_heads);
    a.head_dim = (uint32_t)head_dim;
    a.scale_log2 = (float)(1.4426950408889634 / __builtin_sqrt((double)head_dim));
    a.whole_ok = 1;  // as attn_decode without node handles
    const DecodePlan pr = replan_decode(a, device);
    if (pr.path < 1 || pr.path > 3 || pr.nstate != p.nstate) return (int)hipErrorInvalidValue;
    e = launch_decode_split(a, pr, stream, false);
    if (e != hipSuccess || pr.whole) return (int)e;
    return (int)launch_decode_merge(a, stream, false);
}
