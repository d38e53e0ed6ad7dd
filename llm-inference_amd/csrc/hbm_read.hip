// Measurement helpers for bench.py (libattn_bench.so, not part of the
// attention library): an empty kernel (the launch floor), and a plain
// streaming read of two device buffers, the ceiling a decode call over the
// same K and V bytes can approach.  Every
// byte is loaded once with 16-byte non-temporal loads (the decode's own load
// width and cache hint) and folded into an XOR that is stored only when it
// equals a value the synthetic data never produces, so the loads cannot be
// removed.  Grid: `wgs` workgroups of 512 threads; workgroup i reads the i-th
// of `wgs` equal contiguous slices of A followed by the same slice of B, as a
// decode split workgroup reads its chunk of K and V.
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ u32x4 fold_slice(const u32x4* p, size_t begin, size_t end) {
    constexpr int kUnroll = 8;
    u32x4 acc = {0u, 0u, 0u, 0u};
    for (size_t base = begin + threadIdx.x; base < end; base += 512u * kUnroll) {
        u32x4 v[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const size_t i = base + (size_t)u * 512u;
            v[u] = i < end ? __builtin_nontemporal_load(p + i) : u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) acc ^= v[u];
    }
    return acc;
}

__global__ __launch_bounds__(512) void hbm_read2(const u32x4* a, size_t na, const u32x4* b,
                                                 size_t nb, uint32_t* sink) {
    const size_t wgs = gridDim.x;
    const size_t i = blockIdx.x;
    u32x4 acc = fold_slice(a, na * i / wgs, na * (i + 1) / wgs);
    acc ^= fold_slice(b, nb * i / wgs, nb * (i + 1) / wgs);
    if (acc.x == 0x9e3779b9u && acc.y == 0x7f4a7c15u && acc.z == 0xf39cc060u) sink[0] = acc.w;
}

// The launch floor: a kernel that does no work (its one store is taken only
// when `key` equals a value bench.py never passes), timed like the short
// prompts' kernels to show the fixed cost of a dependent launch in a graph.
__global__ __launch_bounds__(256) void empty_kernel(uint32_t* sink, uint32_t key) {
    if (key == 0x9e3779b9u && threadIdx.x == 0) sink[blockIdx.x] = key;
}

}  // namespace

extern "C" {

// `wgs` workgroups of 256 threads of the empty kernel on `stream`; sink must
// hold `wgs` words (never written for key != 0x9e3779b9).
int attn_bench_empty(uint32_t* sink, unsigned wgs, unsigned key, hipStream_t stream) {
    if (!sink || wgs == 0) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(empty_kernel, dim3(wgs), dim3(256), 0, stream, sink, key);
    return (int)hipGetLastError();
}

// Reads a_bytes at a and b_bytes at b (multiples of 16, 16-byte aligned) on
// `stream`.  Returns a hipError_t as int.
int attn_bench_read2(const void* a, size_t a_bytes, const void* b, size_t b_bytes,
                     uint32_t* sink, unsigned wgs, hipStream_t stream) {
    if (!a || !b || !sink || wgs == 0 || (a_bytes | b_bytes) % 16 ||
        ((uintptr_t)a | (uintptr_t)b) % 16)
        return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(hbm_read2, dim3(wgs), dim3(512), 0, stream,
                       reinterpret_cast<const u32x4*>(a), a_bytes / 16,
                       reinterpret_cast<const u32x4*>(b), b_bytes / 16, sink);
    return (int)hipGetLastError();
}

}  // extern "C"
