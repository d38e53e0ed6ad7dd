// Decode-step QKV projection for gfx950, optionally with the RoPE + KV-cache
// append of the same step folded into its epilogue.
//
// Reference semantics: launch_qkv_decode (qkv_gemm.hip.cpp:107-116) is the
// GEMV y = W x of matrix_vec_mul.hip.cpp:79-172 with beta = 0 (the unfused
// kernel also serves launch_attention_out_projection_decode,
// attention_out_projection.hip.cpp:61-71: the same GEMV with y += beta * y,
// beta = 1 for the residual add): W row-major
// [out_dim][in_dim] (the Q rows of all heads, then K, then V), x [in_dim],
// fp32 accumulation, y rounded to fp16.  In a decode step the engine then runs
// launch_rope_and_store_kv on y (model_inference.hpp:354-369): Q heads rotated
// in place, K rotated into cache row start_pos (y's K left unrotated), V
// copied; NoPE layers copy K and V only.
//
// One wave computes the two output rows of one rotation pair, rows i and
// i + D/2 of a head, so the fused epilogue can rotate them without any
// exchange: 16-byte loads of both weight rows and of x through range-checked
// buffer resources (the tail of a row that is not a multiple of 512 elements
// reads zeros; rows of other lengths or alignments take an element-wise loop), v_dot2_f32_f16 products into fp32 accumulators, a wave
// reduction, then y rounded to fp16 exactly as the GEMV stores it.  The fused
// epilogue applies the rope.hip.cpp:44-58 rotation to those fp16 values (fp32
// products each rounded, no contraction), so its Q, K and cache rows equal the
// two-kernel sequence's bit for bit.  HBM-bound: 2 * out_dim * in_dim bytes of
// weights per call (12.6 MB for SmolLM3, hidden 2048 -> 3072).
#include "attn_internal.hpp"

namespace attn {

namespace {

constexpr int kWavesPerBlock = 4;

// VEC: 16-byte loads (in_dim % 8 == 0, x and W 16-byte aligned); otherwise
// one fp16 element per lane per step, for any length and alignment.
template <bool FUSED, bool VEC>
__global__ __launch_bounds__(64 * kWavesPerBlock) void qkv_gemv(QkvArgs a) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t pair =
        blockIdx.x * kWavesPerBlock + (uint32_t)__builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t npairs = (a.out_dim + 1u) >> 1;
    if (pair >= npairs) return;  // wave-uniform
    const uint32_t D = a.head_dim, half = D >> 1;
    // rows of this wave: a rotation pair when fused, two adjacent rows otherwise
    const uint32_t head = FUSED ? pair / half : 0u;
    const uint32_t i = FUSED ? pair - head * half : 0u;
    const uint32_t row0 = FUSED ? head * D + i : 2u * pair;
    const uint32_t row1 = FUSED ? row0 + half : row0 + 1u;

    const bool has_row1 = row1 < a.out_dim;  // false only for the last row of an odd out_dim
    float acc0 = 0.f, acc1 = 0.f;
    if (VEC) {
        const uint32_t row_bytes = a.in_dim * 2u;
        const BufRsrc rx = make_rsrc(a.x, row_bytes);
        const BufRsrc rw0 = make_rsrc(a.w + (uint64_t)row0 * a.in_dim, row_bytes);
        // a missing second row reads zeros through an empty range
        const BufRsrc rw1 = make_rsrc(a.w + (uint64_t)row1 * a.in_dim, has_row1 ? row_bytes : 0u);
        // 16-byte chunks c = lane + 64 k; all loads of a round are issued first
        constexpr int kRound = 4;
        for (uint32_t base = 0; base < a.in_dim; base += 64u * 8u * kRound) {
            f16x8 xv[kRound], w0[kRound], w1[kRound];
#pragma unroll
            for (int k = 0; k < kRound; ++k) {
                const uint32_t off = (base + (lane + 64u * (uint32_t)k) * 8u) * 2u;
                xv[k] = buf_ld16(rx, off);
                w0[k] = buf_ld16_nt(rw0, off);  // each weight is read once per call
                w1[k] = buf_ld16_nt(rw1, off);
            }
#pragma unroll
            for (int k = 0; k < kRound; ++k)
#pragma unroll
                for (int e = 0; e < 8; e += 2) {
                    const f16x2 xx = {xv[k][e], xv[k][e + 1]};
                    acc0 = __builtin_amdgcn_fdot2(f16x2{w0[k][e], w0[k][e + 1]}, xx, acc0, false);
                    acc1 = __builtin_amdgcn_fdot2(f16x2{w1[k][e], w1[k][e + 1]}, xx, acc1, false);
                }
        }
    } else {
        const f16* w0 = a.w + (uint64_t)row0 * a.in_dim;
        const f16* w1 = a.w + (uint64_t)(has_row1 ? row1 : row0) * a.in_dim;
        for (uint32_t c = lane; c < a.in_dim; c += 64u) {
            const float xc = (float)a.x[c];
            acc0 += (float)w0[c] * xc;
            acc1 += (float)w1[c] * xc;
        }
    }
    // wave sums on the VALU (DPP + lane swaps): the reduction is the tail of
    // every row pair's critical path
    acc0 = wave_sum(acc0);
    acc1 = wave_sum(acc1);
    if (lane != 0) return;
    if (!FUSED) {
        // matrix_vec_mul.hip.cpp:156-163: the fp32 sum plus beta * y, rounded once
        if (a.beta != 0.f) {
            acc0 += a.beta * (float)a.y[row0];
            if (has_row1) acc1 += a.beta * (float)a.y[row1];
        }
        a.y[row0] = (f16)acc0;
        if (has_row1) a.y[row1] = (f16)acc1;
        return;
    }
    const f16 y0 = (f16)acc0;
    const f16 y1 = (f16)acc1;
    // fused RoPE + KV append on the fp16 GEMV outputs
    f16 r0 = y0, r1 = y1;
    if (a.apply) {
#pragma clang fp contract(off)
        const uint64_t t = (uint64_t)a.start_pos * half + i;
        const float c = (float)a.cos_t[t];
        const float s = (float)a.sin_t[t];
        const float x0 = (float)y0, x1 = (float)y1;
        const float p0 = x0 * c;
        const float p1 = x1 * s;
        const float p2 = x1 * c;
        const float p3 = x0 * s;
        r0 = (f16)(p0 - p1);
        r1 = (f16)(p2 + p3);
    }
    const uint64_t kv_dim = (uint64_t)a.num_kv_heads * D;
    if (head < a.num_heads) {  // Q: rotated in place (untouched by NoPE)
        a.y[row0] = r0;
        a.y[row1] = r1;
    } else if (head < a.num_heads + a.num_kv_heads) {  // K: y unrotated, cache rotated
        a.y[row0] = y0;
        a.y[row1] = y1;
        f16* kc = a.kc + (uint64_t)a.start_pos * kv_dim + (uint64_t)(head - a.num_heads) * D;
        kc[i] = r0;
        kc[i + half] = r1;
    } else {  // V: copied
        a.y[row0] = y0;
        a.y[row1] = y1;
        f16* vc = a.vc + (uint64_t)a.start_pos * kv_dim +
                  (uint64_t)(head - a.num_heads - a.num_kv_heads) * D;
        vc[i] = y0;
        vc[i + half] = y1;
    }
}

}  // namespace

bool qkv_vectorized(const QkvArgs& a) {
    const auto a16 = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
    return a.in_dim > 0 && a.in_dim % 8u == 0 && a.in_dim <= 0x7fffffffu && a16(a.x) && a16(a.w);
}

const void* qkv_kernel_symbol(bool fused, bool vec) {
    if (fused)
        return vec ? reinterpret_cast<const void*>(&qkv_gemv<true, true>)
                   : reinterpret_cast<const void*>(&qkv_gemv<true, false>);
    return vec ? reinterpret_cast<const void*>(&qkv_gemv<false, true>)
               : reinterpret_cast<const void*>(&qkv_gemv<false, false>);
}

hipError_t launch_qkv_kernel(const QkvArgs& a, bool fused, hipStream_t stream) {
    const uint32_t npairs = (a.out_dim + 1u) >> 1;
    const dim3 grid((npairs + kWavesPerBlock - 1) / kWavesPerBlock), block(64 * kWavesPerBlock);
    const bool vec = qkv_vectorized(a);
    if (fused && vec)
        hipLaunchKernelGGL((qkv_gemv<true, true>), grid, block, 0, stream, a);
    else if (fused)
        hipLaunchKernelGGL((qkv_gemv<true, false>), grid, block, 0, stream, a);
    else if (vec)
        hipLaunchKernelGGL((qkv_gemv<false, true>), grid, block, 0, stream, a);
    else
        hipLaunchKernelGGL((qkv_gemv<false, false>), grid, block, 0, stream, a);
    return hipGetLastError();
}

}  // namespace attn
