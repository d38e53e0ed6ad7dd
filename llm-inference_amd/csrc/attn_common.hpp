// Shared device/host helpers for the gfx950 (CDNA4, wave64) attention path.
// All kernels in this library are written for wave64 and gfx950's MFMA
// instruction set; nothing here targets another architecture.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace attn {

typedef _Float16 f16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

// 16-byte global load/store of eight fp16 values (pointer must be 16B aligned).
__device__ __forceinline__ f16x8 ld16(const f16* p) {
    return *reinterpret_cast<const f16x8*>(p);
}
__device__ __forceinline__ void st16(f16* p, f16x8 v) {
    *reinterpret_cast<f16x8*>(p) = v;
}
// The same store with the non-temporal hint (the RoPE + KV append kernel's
// outputs: 18.0 -> 16.8 us at 8192 tokens).
__device__ __forceinline__ void st16_nt(f16* p, f16x8 v) {
    __builtin_nontemporal_store(v, reinterpret_cast<f16x8*>(p));
}

// Raw buffer resource over [base, base + bytes): 16-byte loads through it use
// 32-bit offsets, and any load past `bytes` returns zeros without touching
// memory (the gfx9 buffer range check), which replaces per-row clamps.
// dword3 = 0x00020000 selects the 32-bit data format of an untyped buffer.
typedef __amdgpu_buffer_rsrc_t BufRsrc;
__device__ __forceinline__ BufRsrc make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                             0x00020000);
}
__device__ __forceinline__ f16x8 buf_ld16(BufRsrc r, uint32_t byte_off) {
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)byte_off, 0, 0);
    return __builtin_bit_cast(f16x8, v);
}
// The same load with the non-temporal hint (cache-policy bit nt), for data
// that is read exactly once: the decode's K/V stream reads HBM ~10 % faster
// with it (the caches do not keep lines nobody reads again).
__device__ __forceinline__ f16x8 buf_ld16_nt(BufRsrc r, uint32_t byte_off) {
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)byte_off, 0, 2);
    return __builtin_bit_cast(f16x8, v);
}

// One LDS-DMA instruction (buffer_load_dwordx4 ... lds): each lane copies 16
// bytes at byte offset voff of the buffer described by `r` to LDS bytes
// [lds + 16 lane, lds + 16 lane + 16).  Issued as inline assembly so that the
// compiler adds no waits of its own before LDS reads of other buffers (its
// tracking of DMA targets falls back to waiting for every DMA in flight);
// callers await completion explicitly (vmcnt, then a barrier).  M0, the LDS
// base of the instruction, is saved and restored around it.  The resource is
// four SGPRs: base, base >> 32 (stride 0), size in bytes (reads past it return
// zero without touching memory), 0x00020000 (32-bit untyped data).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ u32x4 rsrc_words(const void* base, uint32_t bytes) {
    const uint64_t p = reinterpret_cast<uint64_t>(base);
    return u32x4{(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)p),
                 (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(p >> 32)) & 0xffffu,
                 (uint32_t)__builtin_amdgcn_readfirstlane(bytes), 0x00020000u};
}
__device__ __forceinline__ void dma16(u32x4 r, uint32_t lds, uint32_t voff) {
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %1\n\t"
        "s_nop 0\n\t"
        "buffer_load_dwordx4 %2, %3, 0 offen lds\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "s"(lds), "v"(voff), "s"(r)
        : "memory");
}
// LDS byte address of a pointer into a __shared__ array.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)reinterpret_cast<uintptr_t>(
        (__attribute__((address_space(3))) const char*)(
            __attribute__((address_space(3))) const void*)p);
}

// Cross-lane exchange inside a wave64 (ds_bpermute based).
__device__ __forceinline__ float xor_lane(float v, int mask) {
    return __shfl_xor(v, mask, kWave);
}

// x and the value of lane i ^ 16 (ROWS = 16) or i ^ 32 (ROWS = 32), in one
// order or the other, from one VALU lane swap (v_permlane16_swap_b32 /
// v_permlane32_swap_b32: the odd 16-lane rows of the first operand trade
// places with the even rows of the second, or the upper half of the first
// with the lower half of the second) instead of an LDS-unit permute with its
// ~100 cycles of latency.  The second operand goes through an empty asm so
// the compiler does not take the two operands, and then the two results,
// for the same value.
template <int ROWS>
__device__ __forceinline__ f32x2 lane_swap_pair(float x) {
    float y = x;
    asm volatile("" : "+v"(y));
    const uint32_t a = __builtin_bit_cast(uint32_t, x), b = __builtin_bit_cast(uint32_t, y);
    if constexpr (ROWS == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(a, b, false, false);
        return f32x2{__builtin_bit_cast(float, (uint32_t)r[0]), __builtin_bit_cast(float, (uint32_t)r[1])};
    } else {
        static_assert(ROWS == 32, "lane swaps of 16 or 32 lanes");
        const auto r = __builtin_amdgcn_permlane32_swap(a, b, false, false);
        return f32x2{__builtin_bit_cast(float, (uint32_t)r[0]), __builtin_bit_cast(float, (uint32_t)r[1])};
    }
}
// max / sum of x and lane i ^ MASK's x (MASK 16 or 32); fmaxf and a single
// fp32 add are commutative, so the results equal fmaxf(x, xor_lane(x, MASK))
// and x + xor_lane(x, MASK) bit for bit
template <int MASK>
__device__ __forceinline__ float max_xor(float x) {
    const f32x2 p = lane_swap_pair<MASK>(x);
    return fmaxf(p[0], p[1]);
}
template <int MASK>
__device__ __forceinline__ float add_xor(float x) {
    const f32x2 p = lane_swap_pair<MASK>(x);
    return p[0] + p[1];
}

// Reductions over the 64 lanes of a wave with a uniform result, for a wave
// whose cross-lane steps sit on its critical path: two DPP quad permutes
// (xor 1, xor 2) and two DPP row rotations (by 4 and 8 lanes) reduce each
// 16-lane row into its every lane, then two lane swaps (16, then 32 lanes)
// combine the rows as (r0 op r1) op (r2 op r3) in every lane (against four
// lane reads into scalars: merge kernel 0.04-0.08 us per call faster).  Each
// step is a VALU instruction (a few cycles) where an xor shuffle is an
// LDS-unit permute (~100 cycles of latency).  The result is the same in
// every lane and does not depend on the lane's position.  All 64 lanes must
// be active.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
        0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}
constexpr int kDppXor1 = 0xB1;   // quad_perm [1, 0, 3, 2]
constexpr int kDppXor2 = 0x4E;   // quad_perm [2, 3, 0, 1]
constexpr int kDppRor4 = 0x124;  // row_ror:4
constexpr int kDppRor8 = 0x128;  // row_ror:8
__device__ __forceinline__ float wave_max(float x) {
    x = fmaxf(x, dpp_f<kDppXor1>(x));
    x = fmaxf(x, dpp_f<kDppXor2>(x));
    x = fmaxf(x, dpp_f<kDppRor4>(x));
    x = fmaxf(x, dpp_f<kDppRor8>(x));
    return max_xor<32>(max_xor<16>(x));
}
__device__ __forceinline__ float wave_sum(float x) {
    x += dpp_f<kDppXor1>(x);
    x += dpp_f<kDppXor2>(x);
    x += dpp_f<kDppRor4>(x);
    x += dpp_f<kDppRor8>(x);
    return add_xor<32>(add_xor<16>(x));
}

// 2^x on the hardware transcendental unit (v_exp_f32).  Softmax is computed
// in the log2 domain: scores are pre-multiplied by log2(e)/sqrt(D).
__device__ __forceinline__ float fast_exp2(float x) {
    return __builtin_amdgcn_exp2f(x);
}

constexpr float kLog2e = 1.4426950408889634f;

// RoPE rotation of 8 pairs (x0[i], x1[i]) = (x[c + i], x[c + D/2 + i]) by
// (cos, sin) as rope.hip.cpp:44-58 computes it: fp32 products each rounded,
// no contraction, one fp16 rounding per output.
__device__ __forceinline__ void rope_rotate8(const f16x8 x0, const f16x8 x1, const f16x8 c,
                                             const f16x8 s, f16x8& o0, f16x8& o1) {
#pragma clang fp contract(off)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float a = (float)x0[i];
        const float b = (float)x1[i];
        const float cc = (float)c[i];
        const float ss = (float)s[i];
        const float p0 = a * cc;
        const float p1 = b * ss;
        const float p2 = b * cc;
        const float p3 = a * ss;
        o0[i] = (f16)(p0 - p1);
        o1[i] = (f16)(p2 + p3);
    }
}

}  // namespace attn
