// Fused rotate-half RoPE + FP16 KV-cache append for gfx950.
//
// Semantics follow the reference launcher rope.hip.cpp:138-196 and kernels
// rope.hip.cpp:9-134: token t uses table row start_pos + t; Q heads are
// rotated in place; K heads are rotated into cache row start_pos + t (the K
// source stays unchanged) and V heads copied to the same row; with a null K
// cache K is rotated in place and V is left alone (launch_rope); with
// apply == 0 (NoPE layers) K and V are copied and Q is untouched.
// Rotation: out0 = x0*c - x1*s, out1 = x1*c + x0*s on the pair (i, i + D/2)
// in fp32 with every product rounded (no FMA contraction), then RNE to fp16
// (rope.hip.cpp:44-58).
//
// Vector path (HBM-bound, 12 544 B moved per SmolLM3 token): one lane owns 8
// rotation pairs of one head = a 16-byte load from each half of the head, plus
// the matching 16 bytes of cos and sin.  Per token the lanes cover
// (Hq + 2*Hkv) heads x D/16 lanes, so consecutive lanes stream consecutive
// 16-byte chunks of the [Q | K | V] rows.  Stores carry the non-temporal hint
// (each output byte is written once).
#include "attn_internal.hpp"

namespace attn {

namespace {

__global__ __launch_bounds__(256) void rope_store_kv_vec(RopeArgs a) {
    const uint32_t lanes = a.lanes_per_head;
    const uint32_t slots = a.num_heads + 2u * a.num_kv_heads;
    const uint32_t per_token = slots * lanes;
    const uint32_t gid = blockIdx.x * 256u + threadIdx.x;
    const uint32_t t = gid / per_token;
    if (t >= a.seq_len) return;
    const uint32_t rem = gid - t * per_token;
    const uint32_t slot = rem / lanes;
    const uint32_t j = rem - slot * lanes;
    const uint32_t D = a.head_dim;
    const uint32_t half = D >> 1;
    const uint32_t off0 = j * 8u;
    const uint32_t off1 = half + j * 8u;
    const uint64_t pos = (uint64_t)a.start_pos + t;
    const uint64_t kv_dim = (uint64_t)a.num_kv_heads * D;

    if (slot < a.num_heads) {
        if (!a.apply) return;
        f16* x = a.q + (uint64_t)t * a.q_stride + (uint64_t)slot * D;
        const f16x8 c = ld16(a.cos_t + pos * half + off0);
        const f16x8 s = ld16(a.sin_t + pos * half + off0);
        f16x8 o0, o1;
        rope_rotate8(ld16(x + off0), ld16(x + off1), c, s, o0, o1);
        st16_nt(x + off0, o0);
        st16_nt(x + off1, o1);
        return;
    }
    if (slot < a.num_heads + a.num_kv_heads) {
        const uint32_t h = slot - a.num_heads;
        f16* src = a.k + (uint64_t)t * a.k_stride + (uint64_t)h * D;
        if (a.apply) {
            f16* dst = a.kc ? a.kc + pos * kv_dim + (uint64_t)h * D : src;
            const f16x8 c = ld16(a.cos_t + pos * half + off0);
            const f16x8 s = ld16(a.sin_t + pos * half + off0);
            f16x8 o0, o1;
            rope_rotate8(ld16(src + off0), ld16(src + off1), c, s, o0, o1);
            st16_nt(dst + off0, o0);
            st16_nt(dst + off1, o1);
        } else {
            if (!a.kc) return;
            f16* dst = a.kc + pos * kv_dim + (uint64_t)h * D;
            st16_nt(dst + off0, ld16(src + off0));
            st16_nt(dst + off1, ld16(src + off1));
        }
        return;
    }
    // V head: copied only when a cache is given (launch_rope leaves V alone).
    if (!a.kc) return;
    const uint32_t h = slot - a.num_heads - a.num_kv_heads;
    const f16* src = a.v + (uint64_t)t * a.k_stride + (uint64_t)h * D;
    f16* dst = a.vc + pos * kv_dim + (uint64_t)h * D;
    st16_nt(dst + off0, ld16(src + off0));
    st16_nt(dst + off1, ld16(src + off1));
}

// Generic path: any even head_dim, any strides/alignment.  One thread per
// (token, head slot, pair).  Same arithmetic as the vector path.
__global__ __launch_bounds__(256) void rope_store_kv_generic(RopeArgs a) {
    const uint32_t D = a.head_dim;
    const uint32_t half = D >> 1;
    const uint32_t slots = a.num_heads + 2u * a.num_kv_heads;
    const uint64_t per_token = (uint64_t)slots * half;
    const uint64_t gid = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    const uint64_t t = gid / per_token;
    if (t >= a.seq_len) return;
    const uint64_t rem = gid - t * per_token;
    const uint32_t slot = (uint32_t)(rem / half);
    const uint32_t i = (uint32_t)(rem - (uint64_t)slot * half);
    const uint64_t pos = (uint64_t)a.start_pos + t;
    const uint64_t kv_dim = (uint64_t)a.num_kv_heads * D;

    auto rot = [&](const f16* src, f16* dst) {
#pragma clang fp contract(off)
        const float c = (float)a.cos_t[pos * half + i];
        const float s = (float)a.sin_t[pos * half + i];
        const float x0 = (float)src[i];
        const float x1 = (float)src[i + half];
        const float p0 = x0 * c;
        const float p1 = x1 * s;
        const float p2 = x1 * c;
        const float p3 = x0 * s;
        dst[i] = (f16)(p0 - p1);
        dst[i + half] = (f16)(p2 + p3);
    };

    if (slot < a.num_heads) {
        if (!a.apply) return;
        f16* x = a.q + t * a.q_stride + (uint64_t)slot * D;
        rot(x, x);
        return;
    }
    if (slot < a.num_heads + a.num_kv_heads) {
        const uint32_t h = slot - a.num_heads;
        f16* src = a.k + t * a.k_stride + (uint64_t)h * D;
        if (a.apply) {
            f16* dst = a.kc ? a.kc + pos * kv_dim + (uint64_t)h * D : src;
            rot(src, dst);
        } else if (a.kc) {
            f16* dst = a.kc + pos * kv_dim + (uint64_t)h * D;
            dst[i] = src[i];
            dst[i + half] = src[i + half];
        }
        return;
    }
    if (!a.kc) return;
    const uint32_t h = slot - a.num_heads - a.num_kv_heads;
    const f16* src = a.v + t * a.k_stride + (uint64_t)h * D;
    f16* dst = a.vc + pos * kv_dim + (uint64_t)h * D;
    dst[i] = src[i];
    dst[i + half] = src[i + half];
}

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace

bool rope_vector_ok(const RopeArgs& a) {
    if (a.head_dim % 16 != 0) return false;
    if (a.q_stride % 8 != 0 || a.k_stride % 8 != 0) return false;
    if (!aligned16(a.q) || !aligned16(a.k) || !aligned16(a.cos_t) || !aligned16(a.sin_t)) return false;
    if (a.kc && (!aligned16(a.kc) || !aligned16(a.vc) || !aligned16(a.v))) return false;
    const uint64_t lanes = (uint64_t)a.seq_len * (a.num_heads + 2ull * a.num_kv_heads) * (a.head_dim / 16);
    return lanes < (1ull << 31);
}

const void* rope_kernel_symbol(bool vector_path) {
    return vector_path ? reinterpret_cast<const void*>(&rope_store_kv_vec)
                       : reinterpret_cast<const void*>(&rope_store_kv_generic);
}

hipError_t launch_rope_kernel(const RopeArgs& a, bool vector_path, hipStream_t stream) {
    const uint64_t slots = a.num_heads + 2ull * a.num_kv_heads;
    uint64_t threads;
    if (vector_path) {
        threads = (uint64_t)a.seq_len * slots * a.lanes_per_head;
    } else {
        threads = (uint64_t)a.seq_len * slots * (a.head_dim / 2);
    }
    const uint64_t blocks = (threads + 255) / 256;
    if (blocks == 0) return hipSuccess;
    if (blocks > 0x7fffffffull) return hipErrorInvalidValue;
    if (vector_path) {
        hipLaunchKernelGGL(rope_store_kv_vec, dim3((uint32_t)blocks), dim3(256), 0, stream, a);
    } else {
        hipLaunchKernelGGL(rope_store_kv_generic, dim3((uint32_t)blocks), dim3(256), 0, stream, a);
    }
    return hipGetLastError();
}

}  // namespace attn
