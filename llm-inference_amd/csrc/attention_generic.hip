// Generic grouped-query attention for shapes the MFMA paths do not cover
// (head_dim != 128, unaligned or odd strides, e.g. the reference's Flash-Decode
// known-answer test with D = 32 and kv_stride = kv_dim + 17).
//
// One 256-thread workgroup per (query row, query head).  Keys are streamed in
// tiles of 256: each thread scores one key (fp32 dot product), the tile maximum
// updates the running maximum, and thread d (< D) accumulates sum_j p_j V[j][d].
// Masking follows causal_attention.hip.cpp:177: key j is visible when
// j < kv_len and, for causal rows, j <= row.  Decode calls this with nq = 1 and
// causal = 0 (all kv_len keys visible, causal_attention.hip.cpp:943).
#include "attn_internal.hpp"

namespace attn {

namespace {

constexpr int kTile = 256;

__device__ __forceinline__ float block_max(float v, float* red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    v = red[0];
#pragma unroll
    for (int w = 1; w < kTile / 64; ++w) v = fmaxf(v, red[w]);
    return v;
}

__device__ __forceinline__ float block_sum(float v, float* red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    v = red[0];
#pragma unroll
    for (int w = 1; w < kTile / 64; ++w) v += red[w];
    return v;
}

__global__ __launch_bounds__(kTile) void attention_generic(GenericAttnArgs a) {
    __shared__ float qs[256];
    __shared__ float ps[kTile];
    __shared__ float red[kTile / 64];
    const uint32_t row = blockIdx.x;
    const uint32_t h = blockIdx.y;
    const uint32_t g = h / a.group;
    const uint32_t D = a.head_dim;
    const int tid = threadIdx.x;

    const f16* qrow = a.q + (uint64_t)row * a.q_stride + (uint64_t)h * D;
    if (tid < (int)D) qs[tid] = (float)qrow[tid];
    __syncthreads();

    uint32_t end = a.kv_len;
    if (a.causal && row + 1 < end) end = row + 1;

    float m_run = -INFINITY, l_run = 0.f, acc = 0.f;
    const f16* kb = a.k + (uint64_t)g * D;
    const f16* vb = a.v + (uint64_t)g * D;
    for (uint32_t j0 = 0; j0 < end; j0 += kTile) {
        const uint32_t j = j0 + tid;
        float s = -INFINITY;
        if (j < end) {
            const f16* kr = kb + (uint64_t)j * a.kv_stride;
            float dot = 0.f;
            for (uint32_t d = 0; d < D; ++d) dot += qs[d] * (float)kr[d];
            s = dot * a.scale_log2;
        }
        const float mt = block_max(s, red);
        const float m_new = fmaxf(m_run, mt);
        const float p = (j < end) ? fast_exp2(s - m_new) : 0.f;
        ps[tid] = p;
        const float tile_sum = block_sum(p, red);
        const float alpha = fast_exp2(m_run - m_new);
        l_run = l_run * alpha + tile_sum;
        m_run = m_new;
        if (tid < (int)D) {
            const uint32_t n = (end - j0 < (uint32_t)kTile) ? end - j0 : (uint32_t)kTile;
            float part = 0.f;
            for (uint32_t jj = 0; jj < n; ++jj)
                part += ps[jj] * (float)vb[(uint64_t)(j0 + jj) * a.kv_stride + tid];
            acc = acc * alpha + part;
        }
        __syncthreads();
    }
    if (tid < (int)D) {
        const float o = (end > 0) ? acc / l_run : 0.f;
        a.out[((uint64_t)row * a.num_heads + h) * D + tid] = (f16)o;
    }
}

}  // namespace

const void* generic_attention_symbol() {
    return reinterpret_cast<const void*>(&attention_generic);
}

hipError_t launch_generic_attention(const GenericAttnArgs& a, hipStream_t stream) {
    if (a.head_dim == 0 || a.head_dim > 256 || a.nq == 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(attention_generic, dim3(a.nq, a.num_heads), dim3(kTile), 0, stream, a);
    return hipGetLastError();
}

}  // namespace attn
