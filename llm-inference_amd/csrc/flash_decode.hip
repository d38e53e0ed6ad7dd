// Chunked Flash-Decode for gfx950: single query token, grouped-query heads,
// fp16 KV cache, fp32 softmax, fp16 output.
//
// Reference semantics: causal_attention.hip.cpp:619-716 (per-chunk softmax
// partials) and :719-838 (partial-softmax merge): every key j < kv_len is
// visible; for query head h the KV head is h / (Hq/Hkv); out = softmax(q.K^T /
// sqrt(D)) V in fp32, rounded to fp16.
//
// The context of each KV head is cut into `nsplit` chunks.  A split
// workgroup (8 waves) owns one chunk for HPW KV heads (HPW = 1 up to 12288
// keys, 2 above for SmolLM3); 8/HPW waves share a KV head and each wave
// serves ALL query heads of its group, so every K/V byte is read from HBM
// exactly once (the reference reads it once per query head).  Short
// contexts (up to kWholeMaxKeys) take one chunk per KV head, and that
// workgroup's fold writes the output: one kernel (see plan_decode).
//  * Scores come from v_mfma_f32_16x16x32_f16 as S^T = K . Q^T (keys = rows,
//    the <= 16 grouped query heads = columns): K comes in the A-operand
//    layout either straight from 16-byte loads or, from 4096 keys, through
//    LDS-DMA of whole 256-byte rows.  The S^T key rows are permuted so that lane (gq, n)
//    ends up holding query n and keys 8gq..8gq+7 of a 32-key batch, which is
//    exactly the B-operand layout of P^T for the PV product.
//  * PV is O^T = V^T . P^T on the same MFMA.  Lane (gq, n) loads 16 B of V
//    rows 8gq..8gq+7 at dims 8n..8n+7 (256 B coalesced rows) and transposes
//    the 8x8 block in registers; MFMA tile mt covers dims {8n + mt}, so no
//    LDS round trip is needed, and only the per-query max and sum need
//    cross-lane exchange (two VALU lane swaps, 16 and 32 lanes: C3 14.28
//    against 14.43 us with LDS permutes).  The softmax denominator sums
//    the fp16-rounded P that the PV product multiplies.
//  * K/V are read with the non-temporal hint through raw buffer resources
//    covering exactly the chunk: rows past the chunk read as zero without a
//    memory access, so the last batch needs no clamping and a prefetch past
//    the end is free.  Each wave keeps two 32-key batches in flight: the
//    loads of batch i + 2 are issued as soon as batch i has been consumed.
//  * The waves of a workgroup fold their (max, sum, acc) through LDS into
//    one partial state per query head: fp32 max and sum, and the output
//    normalised by the sum, in fp16.  A chunk of at most two batches is
//    taken by one wave per head, which stores its state from registers.
//
// Two kernels, as in the reference (attention node + merge node): the split
// kernel above writes each workgroup's partial states to the caller's
// workspace, the merge kernel (grid (Hq, D/8), two waves per workgroup, one
// per 4 output dims) folds every split's partial for 4 output dims of one
// head: M = max_c m_c,
// w_c = 2^(m_c-M) l_c, out = sum_c w_c o_c / sum_c w_c.  The kernel
// boundary orders the partial writes before the merge reads.  Measured and
// rejected: one kernel holding the split workgroups and merge workgroups
// (dispatched last) that exchange the partial states through device-coherent
// stores and loads across XCDs -- with a per-split flag (17.3 us per call at
// L = 32768, against 16.5 us for the two kernels), with tagged state words
// polled directly (22.5 us), with system-scope polls (23.3 us): each step of
// the exchange costs a ~1 us memory round trip after the last K/V byte, as
// much as the second launch.
//  * ROPE variants (attn_rope_store_kv_decode): the decode token's RoPE + KV
//    append (rope.hip.cpp:61-134 for one token) folded into the two kernels:
//    the split kernel rotates q in registers and the workgroups whose chunk
//    holds the new row write it before reading their chunk; the merge kernel
//    writes q rotated in place once every split workgroup has read it.
#include "attn_internal.hpp"

#include <algorithm>
#include <type_traits>

namespace attn {

namespace {

constexpr int kD = 128;
constexpr int kMaxSplits = 1024;
// longest context decoded with one KV head per workgroup (see plan_decode)
constexpr uint32_t kOneHeadMaxKeys = 12288;
// shortest context whose split kernel reads K through LDS-DMA (see plan_decode)
constexpr uint32_t kDmaMinKeys = 4096;
// shortest chunk of a split workgroup with two KV heads (see plan_decode)
constexpr uint32_t kTwoHeadMinChunk = 160;
// longest chunk whose batches one wave per head takes (flash_decode_split)
constexpr uint32_t kSoloMaxKeys = 64;
// longest context decoded by one workgroup per KV head (see plan_decode)
constexpr uint32_t kWholeMaxKeys = 384;
constexpr int kAccPitch = kD + 4;
// cache-policy bit nt (non-temporal) of raw buffer loads
constexpr int kNT = 2;

// One 32-key batch in flight: V always in registers; K in registers in the
// MFMA A layout (KDMA = false), or in the wave's LDS tile (KDMA = true).
template <bool KDMA>
struct KVBatch {
    f16x8 k[2][4];
    f16x8 v[8];
};
template <>
struct KVBatch<true> {
    f16x8 v[8];
};

// LDS-DMA of 16 bytes per lane with the non-temporal hint (see dma16)
__device__ __forceinline__ void dma16_nt(u32x4 r, uint32_t lds, uint32_t voff) {
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %1\n\t"
        "s_nop 0\n\t"
        "buffer_load_dwordx4 %2, %3, 0 offen nt lds\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "s"(lds), "v"(voff), "s"(r)
        : "memory");
}

template <int AUX>
__device__ __forceinline__ float buf_ldf(BufRsrc r, uint32_t byte_off) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)byte_off, 0, AUX));
}
template <int AUX>
__device__ __forceinline__ f32x4 buf_ldf4(BufRsrc r, uint32_t byte_off) {
    return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)byte_off, 0, AUX));
}
// every store this lane issued has completed; "memory" keeps the compiler
// from moving stores across
__device__ __forceinline__ void wait_stores() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Timestamps of the instrumented build (libattn_timeline.so, compiled with
// ATTN_DECODE_TIMELINE): TL(...) vanishes from the product library.
#if defined(ATTN_DECODE_TIMELINE)
#define TL(...) __VA_ARGS__
__device__ __forceinline__ uint64_t tl_now() { return __builtin_amdgcn_s_memrealtime(); }
// s_getreg_b32 of HW_ID (hwreg 4, 32 bits) and XCC_ID (hwreg 20, 4 bits)
__device__ __forceinline__ uint64_t tl_hw_id() { return (uint32_t)__builtin_amdgcn_s_getreg(4 | (31 << 11)); }
__device__ __forceinline__ uint64_t tl_xcc_id() { return (uint32_t)__builtin_amdgcn_s_getreg(20 | (3 << 11)); }
#else
#define TL(...)
#endif

// The split kernel: workgroup (grp, c) owns chunk c of KV heads HPW*grp ..
// HPW*grp + HPW-1.  Wave w serves KV head HPW*grp + w % HPW and every
// (8/HPW)-th batch of the chunk, so the waves of a workgroup read whole
// cache-row segments together.  Grid order (decode_grid): while a chunk is at
// most two batches per wave (every load of the call is issued at once) the
// grid is (Hkv / HPW, nsplit), so the head groups of one chunk are
// consecutive workgroups and the round-robin dispatch over the 8 XCDs gives
// each XCD chunks of one head group: 15.65-15.68 against 16.02-16.08 us per
// call at L = 32768 with the chunks consecutive (grid (nsplit, Hkv / HPW),
// each XCD then taking both halves of the same cache rows), level at 254,
// 4096 and 16384 keys.  Longer chunks keep (nsplit, Hkv / HPW): level from
// 40960 to 98304 keys, but 26.3-27.9 against 25.9-26.3 us at 65536.
template <int HPW, bool ROPE, bool KDMA, bool WHOLE>
__global__ __launch_bounds__(512) void flash_decode_split(DecodeArgs a) {
    static_assert(!WHOLE || HPW == 1, "whole-context plans take one KV head per workgroup");
    constexpr int WAVES = 8;
    constexpr int kThreads = WAVES * 64;
    constexpr int kPhases = WAVES / HPW;  // waves sharing one KV head
    const bool head_groups_inner = a.chunk <= 64u * kPhases;
    const uint32_t grp = head_groups_inner ? blockIdx.x : blockIdx.y;
    const uint32_t c = head_groups_inner ? blockIdx.y : blockIdx.x;
    __shared__ float s_m[WAVES][16];
    __shared__ float s_l[WAVES][16];
    // per wave: the fold state (16 x kAccPitch floats); with KDMA it
    // overlays the wave's two K tiles (32 rows x 256 B, one per batch in
    // flight) that LDS-DMA fills, once the wave's last batch is consumed
    constexpr int kWaveLds = KDMA ? 2 * 8192 : 16 * kAccPitch * 4;
    static_assert(16 * kAccPitch * 4 <= kWaveLds);
    __shared__ __attribute__((aligned(16))) char s_w[WAVES][kWaveLds];
    auto sacc = [&](int w, uint32_t q) -> float* {
        return reinterpret_cast<float*>(&s_w[w][0]) + q * kAccPitch;
    };

    // every argument fetched at entry, in one batch: left to the compiler,
    // some were fetched just before the first K/V loads (the score scale,
    // used on both batch paths, the V pointer), whose issue then waited for
    // them (C3 +0.1 us per call)
    asm volatile("" ::"s"(a.q), "s"(a.k), "s"(a.v), "s"(a.kv_stride), "s"(a.kv_len),
                 "s"(a.group), "s"(a.chunk), "s"(a.nstate), "s"(a.scale_log2));
    if constexpr (ROPE)
        asm volatile("" ::"s"(a.q_rot), "s"(a.k_dst), "s"(a.v_dst), "s"(a.k_src), "s"(a.v_src),
                     "s"(a.cos_t), "s"(a.sin_t), "s"(a.row), "s"(a.apply));
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int hw = wave % HPW;
    const int phase = wave / HPW;
    const int n = lane & 15;   // MFMA column (query head in group) / A row
    const int gq = lane >> 4;  // MFMA k-group / output row group
    // The grid is exactly (Hkv / HPW) x nsplit: every launch and every graph
    // node re-plan takes it from decode_grid.  No early exit tests the
    // arguments: a branch on one costs the kernel a kernel-argument round
    // trip before its other argument loads (~0.1 us per call at L = 32768,
    // ~0.05 at 16384 together with the merge kernel's own, see
    // flash_decode_merge_idle).
    TL(const uint64_t tl_t0 = tl_now();
       uint64_t* const tl = a.tl + (uint64_t)(blockIdx.y * gridDim.x + blockIdx.x) * kTlSplitWords;
       if (tid == 0) {
           tl[0] = tl_t0;
           tl[12] = tl_hw_id();
           tl[13] = tl_xcc_id();
       }
       if (lane == 0) tl[2 + wave] = 0;)
    const uint32_t g = grp * HPW + hw;
    const uint32_t G = a.group;
    const uint32_t t0 = c * a.chunk;
    const uint32_t nk = min(a.chunk, a.kv_len - t0);  // keys in this split (>= 1)
    const uint32_t row_bytes = (uint32_t)(a.kv_stride * 2);

    // buffer views of this chunk's K/V rows for KV head g
    const uint32_t span = (nk - 1) * row_bytes + kD * 2;
    const BufRsrc rk = make_rsrc(a.k + (uint64_t)t0 * a.kv_stride + (uint64_t)g * kD, span);
    const BufRsrc rv = make_rsrc(a.v + (uint64_t)t0 * a.kv_stride + (uint64_t)g * kD, span);

    // S^T row m of tile tt is key 8*(m/4) + 4*tt + (m%4) of the batch, so the
    // output of lane group gq is keys 8gq + (4tt + i).
    const uint32_t krow = 8u * (uint32_t)(n >> 2) + (uint32_t)(n & 3);
    // KDMA: K is read like V, 4 whole 256-byte rows per instruction, straight
    // into the wave's LDS tile (32 rows x 256 B): DMA instruction j, lane l
    // loads row r = 4j + l/16, chunk (l % 16) ^ swz(r), into LDS row r, chunk
    // l % 16, where swz(r) = (r & 3) | ((r >> 3) & 3) << 2 = l/16 | 4 (j/2).
    // The 16 rows an A-operand read takes at one chunk then hit 16 distinct
    // bank groups (swz(krow + 4tt) = n).  Otherwise K is loaded in the A
    // layout directly: 16 rows x 64 B per instruction.
    const uint32_t kq = (uint32_t)(lane >> 4);
    uint32_t koff[2];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) koff[tt] = (krow + 4u * tt) * row_bytes + 16u * gq;
    const u32x4 rkw = rsrc_words(a.k + (uint64_t)t0 * a.kv_stride + (uint64_t)g * kD, span);
    const uint32_t kst_base = lds_addr(&s_w[wave][0]);
    uint32_t voff[8];
#pragma unroll
    for (int r = 0; r < 8; ++r) voff[r] = (8u * gq + r) * row_bytes + 16u * n;

    auto load = [&](uint32_t b, KVBatch<KDMA>& kv, int slot) {
        const uint32_t base = b * row_bytes;
        if constexpr (KDMA) {
#pragma unroll
            for (int j = 0; j < 8; ++j)
                dma16_nt(rkw, kst_base + 8192u * slot + 1024u * j,
                         base + (4u * j + kq) * row_bytes +
                             16u * (((uint32_t)lane & 15u) ^ (kq | (4u * (j >> 1)))));
        } else {
#pragma unroll
            for (int tt = 0; tt < 2; ++tt)
#pragma unroll
                for (int s = 0; s < 4; ++s)
                    kv.k[tt][s] = __builtin_bit_cast(
                        f16x8, __builtin_amdgcn_raw_buffer_load_b128(
                                   rk, (int)(base + koff[tt] + 64u * s), 0, kNT));
        }
#pragma unroll
        for (int r = 0; r < 8; ++r)
            kv.v[r] = __builtin_bit_cast(
                f16x8, __builtin_amdgcn_raw_buffer_load_b128(rv, (int)(base + voff[r]), 0, kNT));
    };

    if constexpr (ROPE) {
        // the workgroups whose chunk holds the new token's row append it
        // (K rotated, V copied) and only then read the chunk: the stores are
        // complete (vmcnt) and the barrier orders them before every wave's
        // loads; no other workgroup reads that row's bytes of these heads
        if (a.row >= t0 && a.row - t0 < nk) {
            if (phase == 0 && lane < 16) {
                const uint64_t src = (uint64_t)g * kD;
                const uint64_t dst = (uint64_t)a.row * a.kv_stride + (uint64_t)g * kD;
                if (lane < 8) {  // K: dims 8 lane .. +7 and their partners 64 + 8 lane ..
                    const uint32_t c8 = 8u * (uint32_t)lane;
                    f16x8 k0 = ld16(a.k_src + src + c8), k1 = ld16(a.k_src + src + 64 + c8);
                    if (a.apply)
                        rope_rotate8(k0, k1, ld16(a.cos_t + (uint64_t)a.row * (kD / 2) + c8),
                                     ld16(a.sin_t + (uint64_t)a.row * (kD / 2) + c8), k0, k1);
                    st16(a.k_dst + dst + c8, k0);
                    st16(a.k_dst + dst + 64 + c8, k1);
                } else {         // V: 16 bytes per lane
                    const uint32_t c16 = 16u * (uint32_t)(lane - 8);
                    st16(a.v_dst + dst + c16, ld16(a.v_src + src + c16));
                    st16(a.v_dst + dst + c16 + 8, ld16(a.v_src + src + c16 + 8));
                }
            }
            // the position, for the merge kernel's rotation of q
            if (grp == 0 && hw == 0 && phase == 0 && lane == 16)
                __builtin_amdgcn_raw_buffer_store_b32(a.row, make_rsrc(rope_row_word(a), 4u), 0,
                                                      0, 0);
            wait_stores();
            __syncthreads();
        }
    }
    // a chunk of at most kSoloMaxKeys keys (short contexts): the phase-0
    // wave of each head takes every batch of the chunk (both in flight) and
    // stores the state straight from registers; the other waves have nothing
    // to do (no LDS fold, no barrier)
    const bool solo = a.chunk <= kSoloMaxKeys;
    if (solo && phase != 0) return;

    f32x4 acc[8];
#pragma unroll
    for (int mt = 0; mt < 8; ++mt) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
    // running max: a finite floor, so a wave whose batches all lie past the
    // chunk keeps weight 2^(x - m) = 0 for its masked (-inf) keys and
    // rescale factor 1 without special cases
    float m_run = -1.0e30f;
    float l_run = 0.f;
    // batches b, b + step, ... of the chunk are this wave's
    const uint32_t kStep = solo ? 32u : 32u * kPhases;
    uint32_t b = 32u * phase;
    // wave-uniform: a wave whose first batch lies past the chunk (short
    // contexts) has no keys and goes straight to the fold
    if (b < nk) {
        TL(if (tid == 0) tl[15] = tl_now();)
        // Q^T as the B operand: lane (gq, n) holds Q[g*G + n][32s + 8gq .. +7].
        // Q (and the rotation's cos/sin) are loaded before the first K/V batch so
        // that the in-order load counter never makes a batch wait for them.
        const bool qlane = (uint32_t)n < G;
        f16x8 qb[4], rc[2], rs[2];
        if (qlane) {
            const f16* qp = a.q + (uint64_t)(g * G + n) * kD + 8 * gq;
#pragma unroll
            for (int s = 0; s < 4; ++s) qb[s] = ld16(qp + 32 * s);
            if constexpr (ROPE) {
                const f16* ct = a.cos_t + (uint64_t)a.row * (kD / 2) + 8 * gq;
                const f16* st = a.sin_t + (uint64_t)a.row * (kD / 2) + 8 * gq;
                if (a.apply) {
#pragma unroll
                    for (int s = 0; s < 2; ++s) {
                        rc[s] = ld16(ct + 32 * s);
                        rs[s] = ld16(st + 32 * s);
                    }
                }
            }
        } else {
#pragma unroll
            for (int s = 0; s < 4; ++s) qb[s] = f16x8{};
        }

        KVBatch<KDMA> A, B;
        // after the first loads are issued: q rotated in registers
        auto rotate_q = [&]() {
            TL(if (tid == 0) tl[1] = tl_now();)
            if constexpr (ROPE) {
                // dims 32s + 8gq + i (s = 0, 1) pair with 64 more (s + 2): the
                // lane holds both halves of 16 rotation pairs (rope.hip.cpp:44-58)
                if (qlane && a.apply) {
#pragma unroll
                    for (int s = 0; s < 2; ++s)
                        rope_rotate8(qb[s], qb[s + 2], rc[s], rs[s], qb[s], qb[s + 2]);
                }
            }
        };

        const f16x2 one2 = {(f16)1.0f, (f16)1.0f};

        // this wave's K tile: 32 rows x 256 B in its own slice of s_acc (free
        // until the fold), 16-byte chunk ch of row r at chunk ch ^ swz(r),
        // swz(r) = (r & 3) | ((r >> 3) & 3) << 2, so that the 16 lanes of a
        // row's write and the 16 rows of an A-operand read each cover all 64
        // banks

        // one 32-key batch: scores, online softmax, PV
        // `later`: vector memory operations this wave issued after the batch's
        // K DMAs (its 8 V loads and the other batch's 16 when in flight)
        auto compute = [&](const KVBatch<KDMA>& kv, int slot, uint32_t bb, bool later16) {
            f16x8 ka[2][4];
            if constexpr (KDMA) {
                // the batch's K DMAs have landed: at most the vector memory
                // operations issued after them are outstanding (its 8 V loads,
                // and the other batch's 16 when that one is in flight)
                if (later16)
                    asm volatile("s_waitcnt vmcnt(24)" ::: "memory");
                else
                    asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
                const char* const kst = &s_w[wave][8192 * slot];
#pragma unroll
                for (int tt = 0; tt < 2; ++tt)
#pragma unroll
                    for (int s = 0; s < 4; ++s)  // row krow + 4tt has swz = n
                        ka[tt][s] = *reinterpret_cast<const f16x8*>(
                            kst + (krow + 4u * tt) * 256u +
                            (((uint32_t)(4 * s + gq) ^ (uint32_t)n) << 4));
            } else {
#pragma unroll
                for (int tt = 0; tt < 2; ++tt)
#pragma unroll
                    for (int s = 0; s < 4; ++s) ka[tt][s] = kv.k[tt][s];
            }
            f32x4 st[2];
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
                st[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int s = 0; s < 4; ++s)
                    st[tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka[tt][s], qb[s], st[tt], 0, 0, 0);
            }
            // scores of query n for keys bb + 8gq + r, r = 4tt + i (log2 domain)
            float x[8];
            float mx = -INFINITY;
#pragma unroll
            for (int tt = 0; tt < 2; ++tt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t key = bb + 8u * gq + 4u * tt + i;
                    const float v = (key < nk) ? st[tt][i] * a.scale_log2 : -INFINITY;
                    x[4 * tt + i] = v;
                    mx = fmaxf(mx, v);
                }
            mx = max_xor<16>(mx);
            mx = max_xor<32>(mx);
            const float m_new = fmaxf(m_run, mx);
            const float alpha = fast_exp2(m_run - m_new);
            f16x8 pb;
#pragma unroll
            for (int r = 0; r < 8; ++r) pb[r] = (f16)fast_exp2(x[r] - m_new);
            // the denominator sums the fp16 weights the PV product uses
            float psum = 0.f;
#pragma unroll
            for (int r = 0; r < 4; ++r)
                psum = __builtin_amdgcn_fdot2(f16x2{pb[2 * r], pb[2 * r + 1]}, one2, psum, false);
            l_run = l_run * alpha + psum;
            m_run = m_new;
#pragma unroll
            for (int mt = 0; mt < 8; ++mt) {
                acc[mt] *= alpha;
                f16x8 va;
#pragma unroll
                for (int r = 0; r < 8; ++r) va[r] = kv.v[r][mt];
                acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pb, acc[mt], 0, 0, 0);
            }
        };

        // Batches b, b + kStep, b + 2 kStep, ... of this wave; two in flight:
        // the loads of batch i + 2 go out once batch i is consumed.  Every path
        // into the loop test has exactly batches A and B in flight (the last
        // pair is peeled off below), so the compiler's waits stay vmcnt(16) for
        // A and let B's loads overlap A's compute.  A wave with one batch
        // issues no loads past the chunk (their address processing would still
        // take the CU's load pipeline).  The two forms share no code after
        // their first loads: with a join between a conditional second batch
        // and the first batch's use, the compiler's wait for A would have to
        // cover B as well (the fused RoPE C5 step ran 0.3 us per layer slower).
        if (b + kStep < nk) {
            // the first two batches of this wave
            load(b, A, 0);
            load(b + kStep, B, 1);
            rotate_q();
            while (b + 2 * kStep < nk) {
                __builtin_amdgcn_sched_barrier(0);
                compute(A, 0, b, true);
                load(b + 2 * kStep, A, 0);
                __builtin_amdgcn_sched_barrier(0);
                compute(B, 1, b + kStep, true);
                load(b + 3 * kStep, B, 1);
                b += 2 * kStep;
            }
            __builtin_amdgcn_sched_barrier(0);
            compute(A, 0, b, true);
            __builtin_amdgcn_sched_barrier(0);
            // keys past the chunk are masked (p = 0)
            if (b + kStep < nk) compute(B, 1, b + kStep, false);
        } else {
            load(b, A, 0);
            rotate_q();
            __builtin_amdgcn_sched_barrier(0);
            compute(A, 0, b, false);
        }
        TL(if (lane == 0) tl[2 + wave] = tl_now();)
    }

    // per-query sum over the four lane groups (the max is already shared)
    l_run = add_xor<16>(l_run);
    l_run = add_xor<32>(l_run);
    // whole-context plans with RoPE: this workgroup is the only reader of
    // its query heads, so once every wave has read them it writes them back
    // rotated, as the merge kernel does otherwise (lanes 0..7 of the phase-0
    // wave of KV head g, query heads g G .. g G + G - 1)
    auto store_q_rotated = [&]() {
        if constexpr (ROPE) {
            if (WHOLE && a.apply && phase == 0 && lane < 8)
                for (uint32_t qn = 0; qn < G; ++qn)
                    rotate_q_head(a, g * G + qn, (uint32_t)lane, a.row);
        }
    };
    if (solo) {
        // the split's state is this wave's (what the fold below would give:
        // the other waves of the head carry weight 0); lane (gq, n < G) holds
        // dims 32gq + 8i + mt = acc[mt][i] of query n
        if (WHOLE && (uint32_t)n < G) {
            // the only split: its state is the output
            const float inv = 1.0f / l_run;
            f16* const oh = a.out + (uint64_t)(g * G + n) * kD + 32u * gq;
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int mt = 0; mt < 8; ++mt) oh[8 * i + mt] = (f16)(acc[mt][i] * inv);
        } else if ((uint32_t)n < G) {
            const BufRsrc rpo = make_rsrc(a.part_out, a.num_heads * a.nstate * kD * 2u);
            const uint32_t st = (g * G + (uint32_t)n) * a.nstate + c;
            const float inv = 1.0f / l_run;  // l_run >= 1: the chunk's maximum has weight 1
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                f16x8 o;
#pragma unroll
                for (int mt = 0; mt < 8; ++mt) o[mt] = (f16)(acc[mt][i] * inv);
                __builtin_amdgcn_raw_buffer_store_b128(
                    __builtin_bit_cast(u32x4, o), rpo, (int)((st * kD + 32u * gq + 8u * i) * 2u),
                    0, 0);
            }
            if (gq == 0) {
                a.part_max[st] = m_run;
                a.part_sum[st] = l_run;
            }
        }
        store_q_rotated();  // the other waves returned before reading q
        TL(if (lane == 0) {
               tl[14] = tl[10] = tl_now();
               wait_stores();
               tl[11] = tl_now();
           })
        return;
    }
    // only the G columns that are query heads go to LDS: lane (gq, n < G)
    // holds dims 32gq .. 32gq + 31 of query n (tile mt, row 4gq + i = dim
    // 8(4gq + i) + mt), written as 16-byte rows
    if ((uint32_t)n < G) {
        if (gq == 0) {
            s_m[wave][n] = m_run;
            s_l[wave][n] = l_run;
        }
        float* const sa = sacc(wave, n);
#pragma unroll
        for (int mt = 0; mt < 8; ++mt)
#pragma unroll
            for (int i = 0; i < 4; ++i) sa[32 * gq + 8 * i + mt] = acc[mt][i];
    }
    __syncthreads();
    TL(if (tid == 0) tl[14] = tl_now();)

    // fold the kPhases waves of each KV head and write its partials: thread
    // idx handles 4 consecutive dims of one (head, query) state, stored with
    // one 16-byte buffer store (the range covers this workgroup's head group)
    const uint32_t rows = HPW * G;  // states of this workgroup, (head, query) order
    const BufRsrc rpo = make_rsrc(state_out(a) + (uint64_t)grp * rows * a.nstate * kD,
                                  rows * a.nstate * kD * 2u);
    for (uint32_t idx = tid; idx < rows * (kD / 4); idx += kThreads) {
        const uint32_t row = idx >> 5;  // kD / 4 = 32 items per state
        const uint32_t hl = row / G;
        const uint32_t qn = row - hl * G;
        const uint32_t d = (idx & 31u) * 4u;
        // every LDS read of the item first (one round trip), then the math
        float mw[kPhases], lw[kPhases];
        f32x4 aw[kPhases];
#pragma unroll
        for (int ph = 0; ph < kPhases; ++ph) {
            const int w = hl + HPW * ph;
            mw[ph] = s_m[w][qn];
            lw[ph] = s_l[w][qn];
            aw[ph] = *reinterpret_cast<const f32x4*>(sacc(w, qn) + d);
        }
        float M = mw[0];
#pragma unroll
        for (int ph = 1; ph < kPhases; ++ph) M = fmaxf(M, mw[ph]);
        f32x4 num = {0.f, 0.f, 0.f, 0.f};
        float den = 0.f;
#pragma unroll
        for (int ph = 0; ph < kPhases; ++ph) {
            const float wt = fast_exp2(mw[ph] - M);  // waves without keys: 0
            num += wt * aw[ph];
            den += wt * lw[ph];
        }
        // the state's output normalised by its own sum (den >= 1: the chunk's
        // maximum has weight 1), in fp16
        const float inv = 1.0f / den;
        if constexpr (WHOLE) {
            // the only split: the state is the output of query head
            // (grp HPW + hl) G + qn
            f16* const o = a.out + (uint64_t)((grp * HPW + hl) * G + qn) * kD + d;
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] = (f16)(num[e] * inv);
            continue;
        }
        const uint32_t st = row * a.nstate + c;  // state index within the head group
        const f16x4 o = {(f16)(num[0] * inv), (f16)(num[1] * inv), (f16)(num[2] * inv),
                         (f16)(num[3] * inv)};
        __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, o), rpo,
                                              (int)((st * kD + d) * 2u), 0, 0);
        if (d == 0) {
            const uint64_t sg = (uint64_t)grp * rows * a.nstate + st;
            a.part_max[sg] = M;
            a.part_sum[sg] = den;
        }
    }
    store_q_rotated();  // every wave of this workgroup has read q (barrier above)
    TL(if (tid == 0) {
           tl[10] = tl_now();
           wait_stores();
           tl[11] = tl_now();
       })
}

constexpr int kMergeDims = 4;    // output dims per merge wave
// waves per merge workgroup, each on its own 4 dims: C3 14.56 against 14.63
// us with one wave (512 workgroups), 16384 keys 9.82 against 9.91, 4096 keys
// 5.93 against 5.98; four waves 14.68 us (same box, alternating builds)
constexpr int kMergeWaves = 2;
constexpr int kMergeRound = 4;   // splits per lane per round of loads past 128 states

// The merge kernel: grid (Hq, D/8), two independent waves per workgroup,
// wave w of workgroup (h, y) on dims 4 (2y + w) .. +3 of head h.  Lane j
// folds the partials of splits j, j + 64, ... for 4 output dims of one head
// with an online merge (all loads of a round issued first, through
// range-checked buffer resources: splits past nstate read as zero and get
// weight 0); the 64 lanes then combine with DPP moves and lane swaps
// (wave_max, wave_sum).
template <bool ROPE>
__global__ __launch_bounds__(64 * kMergeWaves) void flash_decode_merge(DecodeArgs a) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t h = blockIdx.x;
    const uint32_t dg = blockIdx.y * kMergeWaves + (threadIdx.x >> 6);
    const uint32_t d0 = dg * kMergeDims;
    const uint32_t S = a.nstate;
    TL(uint64_t* const tl = a.tl + kTlMergeBase + 4u * (uint64_t)(dg * gridDim.x + blockIdx.x);
       if (lane == 0) {
           tl[0] = tl_now();
           tl[3] = tl_xcc_id();
       })
    const BufRsrc rpm = make_rsrc(a.part_max + (uint64_t)h * S, S * 4u);
    const BufRsrc rps = make_rsrc(a.part_sum + (uint64_t)h * S, S * 4u);
    const BufRsrc rpo = make_rsrc(state_out(a) + (uint64_t)h * S * kD, S * kD * 2u);
    const uint32_t dbyte = d0 * 2u;
    // the rotating lanes fetch the position first, alongside the states
    const bool rotates = ROPE && a.apply && dg < 8 && lane == 0;
    uint32_t row = 0;
    if (rotates) row = __hip_atomic_load(rope_row_word(a), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

    float m = -INFINITY, l = 0.f;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    // one round of loads: states base, base + 64, ..., R of them per lane
    auto fold_round = [&](uint32_t base, auto r_tag) __attribute__((always_inline)) {
        constexpr int R = decltype(r_tag)::value;
        float mc[R], lc[R];
        f16x4 ac[R];
#pragma unroll
        for (int u = 0; u < R; ++u) {
            const uint32_t c = base + 64u * (uint32_t)u;
            mc[u] = buf_ldf<0>(rpm, c * 4u);
            lc[u] = buf_ldf<0>(rps, c * 4u);
            ac[u] = __builtin_bit_cast(
                f16x4, __builtin_amdgcn_raw_buffer_load_b64(rpo, (int)(c * (kD * 2u) + dbyte), 0, 0));
        }
#pragma unroll
        for (int u = 0; u < R; ++u)
            if (base + 64u * (uint32_t)u >= S) mc[u] = -INFINITY;
        float mn = m;
#pragma unroll
        for (int u = 0; u < R; ++u) mn = fmaxf(mn, mc[u]);  // split `base` is valid
        const float so = fast_exp2(m - mn);  // first round: 2^-inf = 0
        l *= so;
        acc *= so;
#pragma unroll
        for (int u = 0; u < R; ++u) {
            // state c's weight 2^(m_c - M) l_c times its normalised output
            const float wc = fast_exp2(mc[u] - mn) * lc[u];  // invalid splits: 0
            l += wc;
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[e] += (float)ac[u][e] * wc;
        }
        m = mn;
    };
    // as many loads per lane as the states need, in one round up to 256
    // states (each load past nstate still takes the address pipeline: rounds
    // of 4 at 128 states 14.54 against 14.49 us at C3)
    if (S <= 64u) {
        if (lane < S) fold_round(lane, std::integral_constant<int, 1>{});
    } else if (S <= 128u) {
        fold_round(lane, std::integral_constant<int, 2>{});
    } else {
        for (uint32_t base = lane; base < S; base += 64u * kMergeRound)
            fold_round(base, std::integral_constant<int, kMergeRound>{});
    }
    TL(if (lane == 0) tl[1] = tl_now();)
    // lanes without splits hold m = -inf and get weight 0
    const float mx = wave_max(m);
    const float w = fast_exp2(m - mx);
    const float den = wave_sum(w * l);
    f32x4 num;
#pragma unroll
    for (int e = 0; e < 4; ++e) num[e] = wave_sum(acc[e] * w);
    // every lane holds the sums; lane e writes dim d0 + e (out may be 2-byte aligned)
    if (lane < (uint32_t)kMergeDims) {
        float v = num[0];
#pragma unroll
        for (int e = 1; e < 4; ++e) v = lane == (uint32_t)e ? num[e] : v;
        a.out[(uint64_t)h * kD + d0 + lane] = (f16)(v / den);
    }
    TL(wait_stores(); if (lane == 0) tl[2] = tl_now();)
    if constexpr (ROPE) {
        // every split workgroup has read q (the kernel boundary orders this)
        if (rotates) rotate_q_head(a, h, dg, row);
    }
}

// The merge node of a whole-context plan (the split kernel wrote the output
// and q): nothing to do.  A kernel of its own, so that the merge kernel
// proper tests no flag before its loads (a branch on an argument costs it a
// kernel-argument round trip of its own, ~0.3 us per call at L = 32768).
template <bool ROPE>
__global__ __launch_bounds__(64 * kMergeWaves) void flash_decode_merge_idle(DecodeArgs) {}

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace

int decode_hpw(int path) { return path == 1 ? 4 : path == 2 ? 2 : path == 3 ? 1 : 0; }

template <bool ROPE, bool KDMA>
const void* split_symbol_of(int path, bool whole) {
    if (whole) return path == 3 ? reinterpret_cast<const void*>(
                                      &flash_decode_split<1, ROPE, KDMA, true>)
                                : nullptr;
    if (path == 1) return reinterpret_cast<const void*>(&flash_decode_split<4, ROPE, KDMA, false>);
    if (path == 2) return reinterpret_cast<const void*>(&flash_decode_split<2, ROPE, KDMA, false>);
    if (path == 3) return reinterpret_cast<const void*>(&flash_decode_split<1, ROPE, KDMA, false>);
    return nullptr;
}

// path 1/2/3: 4/2/1 KV heads per workgroup; kdma: K through LDS-DMA; whole:
// the one-split plan whose fold writes the output (path 3 only)
const void* split_symbol(int path, bool rope, bool kdma, bool whole) {
    if (rope)
        return kdma ? split_symbol_of<true, true>(path, whole)
                    : split_symbol_of<true, false>(path, whole);
    if (path < 1 || path > 3) return generic_attention_symbol();
    return kdma ? split_symbol_of<false, true>(path, whole)
                : split_symbol_of<false, false>(path, whole);
}

const void* decode_split_symbol(const DecodePlan& p, bool rope) {
    return split_symbol(p.path, rope, p.kdma != 0, p.whole != 0);
}

const void* decode_merge_symbol(bool rope, bool whole) {
    if (whole)
        return rope ? reinterpret_cast<const void*>(&flash_decode_merge_idle<true>)
                    : reinterpret_cast<const void*>(&flash_decode_merge_idle<false>);
    return rope ? reinterpret_cast<const void*>(&flash_decode_merge<true>)
                : reinterpret_cast<const void*>(&flash_decode_merge<false>);
}

int decode_path_of_symbol(const void* fn, bool rope) {
    for (int path = 1; path <= 3; ++path)
        for (int kdma = 0; kdma < 2; ++kdma)
            for (int whole = 0; whole < 2; ++whole)
                if (fn && fn == split_symbol(path, rope, kdma != 0, whole != 0)) return path;
    return 0;
}

DecodePlan plan_decode(uint32_t kv_len, uint32_t num_heads, uint32_t num_kv_heads,
                       uint32_t head_dim, uint64_t kv_stride, const void* q, const void* k,
                       const void* v, int device, bool allow_whole) {
    DecodePlan p{0, 1, kv_len, 1, 256, 1, 0};
    const uint32_t G = num_heads / num_kv_heads;
    const bool mfma_ok = head_dim == kD && G >= 1 && G <= 16 && kv_stride % 8 == 0 &&
                         kv_stride * 2 <= 0x40000000ull && aligned16(q) && aligned16(k) &&
                         aligned16(v) && get_option(kOptDecodeForceGeneric) == 0;
    if (!mfma_ok) return p;
    // one KV head per workgroup up to kOneHeadMaxKeys keys (SmolLM3: twice
    // the workgroups on a context that does not fill the chip), two above
    // when Hkv allows (fewer partial states to merge)
    uint32_t hpw = (num_kv_heads % 2 == 0 && kv_len > kOneHeadMaxKeys) ? 2 : 1;
    // a forced count is reduced to what Hkv allows
    const long hopt = get_option(kOptDecodeHeadsPerGroup);
    if (hopt == 4 || hopt == 2 || hopt == 1) {
        hpw = (uint32_t)hopt;
        while (num_kv_heads % hpw != 0) hpw /= 2;
    }
    p.path = hpw == 4 ? 1 : hpw == 2 ? 2 : 3;
    p.block = 512;
    const uint32_t groups = num_kv_heads / hpw;
    p.groups = groups;
    // chunks are sized in steps of 8 keys (the waves mask the keys of a
    // partial batch): a step of one batch per wave (32 * 8/HPW keys) left up
    // to a third of the CUs idle just past multiples of 16384 keys (L = 32769:
    // 86 splits of 384 keys, 20.1 us, against 125 of 264 keys, 16.5 us)
    const uint32_t unit = 8u;
    const uint32_t units = (kv_len + unit - 1) / unit;
    const uint32_t cus = (uint32_t)std::max(1, device_cu_count(device));
    const long sopt = get_option(kOptDecodeSplits);
    // one 8-wave workgroup per CU; with two KV heads per workgroup past
    // kOneHeadMaxKeys, chunks of at least kTwoHeadMinChunk keys even if CUs
    // stay idle (L = 16384: 103 splits of 160 keys 10.30 us, 128 of 128 keys
    // 10.79 us; 14336: 9.86 against 10.19 us; equal or better from 13312 to
    // 19456 keys; a forced two-head plan on a short context keeps its splits)
    uint32_t target = sopt > 0 ? (uint32_t)sopt : std::max(1u, (cus + groups - 1) / groups);
    if (sopt <= 0 && hpw == 2 && kv_len > kOneHeadMaxKeys)
        target = std::min(target, std::max(1u, (kv_len + kTwoHeadMinChunk - 1) / kTwoHeadMinChunk));
    uint32_t nsplit = std::max(1u, std::min<uint32_t>({target, units, (uint32_t)kMaxSplits}));
    // at least 16 keys per split: with chunks of >= KV_CHUNK (12) keys the
    // states fit the caller's Hq * ceil(L / 12)-state workspace
    uint32_t chunk = std::max(16u, ((units + nsplit - 1) / nsplit) * unit);
    // a chunk's rows must fit one 32-bit buffer range
    const uint64_t max_rows = (0xffffffffull - kD * 2) / (kv_stride * 2);
    while (chunk > max_rows && chunk > 16u) chunk -= unit;
    nsplit = (kv_len + chunk - 1) / chunk;
    // short contexts, when the caller allows one kernel: one workgroup per
    // KV-head group takes the whole context and its fold writes the output
    // (the merge's kernel boundary and partial-state round trip, ~2.3 us of a
    // 254-key call, are gone).  Its K goes through LDS-DMA in whole rows: the
    // four workgroups are bound by their CUs' load pipelines, which the
    // A-layout reads (16 rows x 64 B per instruction) use half as well
    // (L = 254: 3.81 us against 4.92 us with K in registers and 4.67 us split;
    // 384 keys: 4.48 against 4.67 split)
    const long wopt = get_option(kOptDecodeWholeMaxKeys);
    const uint64_t whole_max = wopt < 0 ? 0u : wopt > 0 ? (uint64_t)wopt : kWholeMaxKeys;
    if (allow_whole && sopt <= 0 && hpw == 1 && kv_len <= whole_max && kv_len <= max_rows) {
        nsplit = 1;
        chunk = (kv_len + unit - 1) / unit * unit;
        p.whole = 1;
    }
    p.nsplit = nsplit;
    p.chunk = chunk;
    p.nstate = nsplit;  // one folded state per split and query head
    // K through LDS-DMA in whole 256-byte rows once the call streams (from
    // kDmaMinKeys keys); below, the call is latency-bound and K goes straight
    // into registers in the MFMA layout, one step shorter per batch
    // (chunks of at most kSoloMaxKeys, which one wave per head takes, keep K
    // in registers: L = 4096, 64-key chunks: 6.35 against 6.60 us)
    const long kopt = get_option(kOptDecodeKdma);
    p.kdma = kopt == 1   ? 0u
             : kopt == 2 ? 1u
                         : ((kv_len >= kDmaMinKeys && chunk > kSoloMaxKeys) || p.whole ? 1u : 0u);
    return p;
}

DecodePlan replan_decode(DecodeArgs& a, int device) {
    const DecodePlan p = plan_decode(a.kv_len, a.num_heads, a.num_kv_heads, a.head_dim,
                                     a.kv_stride, a.q, a.k, a.v, device, a.whole_ok != 0);
    a.nsplit = p.nsplit;
    a.chunk = p.chunk;
    a.nstate = p.nstate;
    a.whole = p.whole;
    return p;
}

// the split kernel's grid: head groups inner while a chunk is at most two
// batches per wave (flash_decode_split derives the same order from a.chunk)
dim3 decode_grid(const DecodeArgs& a, const DecodePlan& p) {
    const uint32_t phases = 8u / (uint32_t)decode_hpw(p.path);
    return a.chunk <= 64u * phases ? dim3(p.groups, a.nsplit) : dim3(a.nsplit, p.groups);
}

// one workgroup per query head and 4 output dims; one workgroup, which
// exits at once, for a whole-context plan
dim3 decode_merge_grid(const DecodeArgs& a) {
    return a.whole ? dim3(1, 1) : dim3(a.num_heads, kD / kMergeDims / kMergeWaves);
}

#if defined(ATTN_DECODE_TIMELINE)
// instrumented build: each split launch takes the next of `tl_slots` records
// (round robin), its merge launch the same one
namespace {
uint64_t* tl_base = nullptr;
uint32_t tl_slots = 0, tl_next = 0, tl_cur = 0;
uint64_t* tl_record(bool next) {
    if (!tl_base || tl_slots == 0) return nullptr;
    if (next) {
        tl_cur = tl_next;
        tl_next = (tl_next + 1) % tl_slots;
    }
    return tl_base + (uint64_t)tl_cur * kTlSlotWords;
}
}  // namespace
#endif

hipError_t launch_decode_split(const DecodeArgs& a, const DecodePlan& p, hipStream_t stream,
                               bool rope) {
    if (p.path < 1 || p.path > 3) return hipErrorInvalidValue;
    const void* fn = decode_split_symbol(p, rope);
#if defined(ATTN_DECODE_TIMELINE)
    DecodeArgs t = a;
    t.tl = tl_record(true);
    const dim3 grid = decode_grid(a, p);
    if (!t.tl || grid.x * grid.y > kTlMaxSplitWgs) return hipErrorInvalidValue;
    void* args[1] = {&t};
    return hipLaunchKernel(fn, grid, dim3(512), args, 0, stream);
#else
    void* args[1] = {const_cast<DecodeArgs*>(&a)};
    return hipLaunchKernel(fn, decode_grid(a, p), dim3(512), args, 0, stream);
#endif
}

hipError_t launch_decode_merge(const DecodeArgs& a, hipStream_t stream, bool rope) {
#if defined(ATTN_DECODE_TIMELINE)
    DecodeArgs t = a;
    t.tl = tl_record(false);
    if (!t.tl || a.num_heads * (kD / kMergeDims) > kTlMaxMergeWgs) return hipErrorInvalidValue;
    void* args[1] = {&t};
#else
    void* args[1] = {const_cast<DecodeArgs*>(&a)};
#endif
    return hipLaunchKernel(decode_merge_symbol(rope, a.whole != 0), decode_merge_grid(a),
                           dim3(64 * kMergeWaves), args, 0, stream);
}

}  // namespace attn

#if defined(ATTN_DECODE_TIMELINE)
// Instrumented build only: decode calls write their timestamps to `slots`
// records of kTlSlotWords 64-bit words at `buf` (device memory), in turn,
// starting with record 0.  Without a buffer the decode launchers refuse.
extern "C" int attn_timeline_set(void* buf, size_t slots) {
    attn::tl_base = static_cast<uint64_t*>(buf);
    attn::tl_slots = (uint32_t)slots;
    attn::tl_next = attn::tl_cur = 0;
    return 0;
}
extern "C" size_t attn_timeline_slot_words() { return attn::kTlSlotWords; }
#endif
