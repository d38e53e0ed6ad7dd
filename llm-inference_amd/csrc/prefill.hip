// Causal grouped-query prefill attention for gfx950 on fp16 MFMA.
//
// Reference semantics: causal_attention.hip.cpp:271-374 with the launcher
// :376-451 -- query t of head h attends to keys 0..t of KV head h/(Hq/Hkv),
// scores q.k/sqrt(D), softmax in fp32, output packed [N][Hq][D] fp16; start
// position 0 and kv_len = N (:388-390).
//
// MFMA path (D = 128, Hq/Hkv a multiple of 4, 16-byte aligned rows):
//  * workgroup = 64 query tokens of 4 query heads sharing one KV head, as 8
//    waves (two per head, 32 queries each, 2 waves per SIMD so one wave's
//    softmax overlaps the other's MFMAs; everything stays in VGPRs) or, as an
//    option, 4 waves of 64 queries (each LDS operand feeds two MFMAs).
//  * K and V of a 64-key tile are staged in LDS once per workgroup and shared
//    by the 4 heads (the reference re-reads them per head).  V is stored
//    transposed (V^T[dim][key]) with the keys of every 16-key MFMA step in the
//    order the S^T accumulator produces them, so P never leaves registers.
//  * S^T = K . Q^T with v_mfma_f32_32x32x16_f16: keys are MFMA rows, queries
//    columns, so each lane holds one query's scores and the online softmax
//    (running max, running sum, rescale) is per lane plus one xor-32 exchange.
//  * O^T = V^T . P^T on the same MFMA; O^T stays in 64 accumulator registers.
//  * Causal tile skipping: query tile i visits key tiles 0..i only; the
//    diagonal tile is masked.  Tiles are handed out longest-first and the
//    four head groups of one KV head are kept on the same pair of XCDs so the
//    KV head's K/V stays in one L2.
//  * K/V tile j+1 is prefetched into registers while tile j is computed; two
//    LDS buffers, one barrier per tile.
#include "attn_internal.hpp"

#include <type_traits>

namespace attn {

namespace {

constexpr int kD = 128;
constexpr int kBM = 64;        // query tokens per workgroup (per wave)
constexpr int kBN = 64;        // keys per tile
constexpr int kKP = kD + 8;    // K tile row pitch (halves): conflict-free 16 B reads
constexpr int kVP = kBN + 8;   // V^T tile row pitch (halves)

__device__ __forceinline__ f16x8 lds16(const f16* p) {
    return *reinterpret_cast<const f16x8*>(p);
}

__device__ __forceinline__ f32x16 mfma32(f16x8 a, f16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// blockIdx -> (head quad, query tile), longest tiles first, head quads pinned
// to XCD subsets (workgroups are dispatched round-robin over the 8 XCDs).
__device__ __forceinline__ bool map_block(uint32_t bid, uint32_t quads, uint32_t q_tiles,
                                          uint32_t& quad, uint32_t& tile) {
    if (quads <= 8 && (8 % quads) == 0) {
        const uint32_t xcd = bid & 7u;
        const uint32_t j = bid >> 3;
        const uint32_t per = 8u / quads;
        quad = xcd % quads;
        const uint32_t rank = j * per + xcd / quads;
        if (rank >= q_tiles) return false;
        tile = q_tiles - 1u - rank;
        return true;
    }
    const uint32_t rank = bid / quads;
    quad = bid - rank * quads;
    if (rank >= q_tiles) return false;
    tile = q_tiles - 1u - rank;
    return true;
}

// Lazy rescaling: the running maximum used for exp2 is only raised when a row
// maximum exceeds it by more than kRescaleSlack (log2 units), so P <= 2^8 in
// fp16 and the O^T accumulators are rarely touched by VALU code.
constexpr float kRescaleSlack = 8.0f;

// NT 32-query column tiles per wave.  NT = 2: 4 waves (one per grouped head,
// 64 queries each, 1 wave per SIMD); NT = 1: 8 waves (two per head, 32
// queries each, 2 waves per SIMD so one wave's softmax overlaps the other's
// MFMAs).  Either way a workgroup covers 64 query tokens of 4 heads.
template <int NT>
__global__ __launch_bounds__(256 * (2 / NT), 1) void prefill_d128(PrefillArgs a) {
    constexpr int kWaves = 4 * (2 / NT);
    constexpr int kThreads = 64 * kWaves;
    constexpr int kKChunks = (kBN * kD / 8) / kThreads;  // 16 B K chunks per thread
    constexpr int kVKeys = (kBN * kD / 8) / kThreads;    // V keys per thread (x 8 dims)
    __shared__ __attribute__((aligned(16))) f16 kt[2][kBN * kKP];
    __shared__ __attribute__((aligned(16))) f16 vt[2][kD * kVP];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: SGPR descriptors
    const int n = lane & 31;   // MFMA column (query) / A-operand row
    const int hh = lane >> 5;  // MFMA k-half / output row half

    const uint32_t quads = a.num_heads / 4u;
    uint32_t quad, tile;
    if (!map_block(blockIdx.x, quads, a.q_tiles, quad, tile)) return;
    const uint32_t head = 4u * quad + (uint32_t)(wave & 3);
    const uint32_t g = (4u * quad) / a.group;
    const uint32_t N = a.seq_len;
    const uint32_t q0 = tile * kBM + 32u * NT * (uint32_t)(wave >> 2);  // this wave's first query
    const uint32_t q_row_bytes = (uint32_t)(a.q_stride * 2);
    const uint32_t kv_row_bytes = (uint32_t)(a.kv_stride * 2);

    // buffer views: rows past N read as zero (no guards needed)
    const BufRsrc rq = make_rsrc(a.q + (uint64_t)head * kD, (N - 1) * q_row_bytes + kD * 2);
    const BufRsrc rk = make_rsrc(a.k + (uint64_t)g * kD, (N - 1) * kv_row_bytes + kD * 2);
    const BufRsrc rv = make_rsrc(a.v + (uint64_t)g * kD, (N - 1) * kv_row_bytes + kD * 2);

    // Q^T B operands: lane (hh, n) of column tile nt holds
    // Q[q0 + 32nt + n][head][16s + 8hh .. +7] for k-step s.
    f16x8 qb[NT][8];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        const uint32_t off = (q0 + 32u * nt + n) * q_row_bytes + 16u * hh;
#pragma unroll
        for (int s = 0; s < 8; ++s) qb[nt][s] = buf_ld16(rq, off + 32u * s);
    }

    f32x16 o[NT][4];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) o[nt][dt] = f32x16{};
    float m_used[NT], l_run[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        m_used[nt] = -INFINITY;
        l_run[nt] = 0.f;
    }

    // global -> register staging of one 64-key tile: K as 16 B chunks, V as
    // kVKeys consecutive keys x 8 dims per thread (transposed on the LDS store)
    constexpr uint32_t kKeyGroups = kBN / kVKeys;
    const uint32_t kgrp = tid % kKeyGroups;  // keys kVKeys*kgrp ..
    const uint32_t dg = tid / kKeyGroups;    // dims 8dg..8dg+7
    f16x8 kr[kKChunks], vr[kVKeys];
    auto gload = [&](uint32_t kv0) {
#pragma unroll
        for (int i = 0; i < kKChunks; ++i) {
            const uint32_t e = (uint32_t)i * kThreads + tid;
            kr[i] = buf_ld16(rk, (kv0 + (e >> 4)) * kv_row_bytes + 16u * (e & 15u));
        }
#pragma unroll
        for (int r = 0; r < kVKeys; ++r)
            vr[r] = buf_ld16(rv, (kv0 + kVKeys * kgrp + r) * kv_row_bytes + 16u * dg);
    };
    // key 16ks + 8b + 4h + r sits in V^T slot ks*16 + h*8 + 4b + r: the order
    // in which S^T tile ks/2 presents keys to PV k-step ks
    const uint32_t key0 = kVKeys * kgrp;
    const uint32_t vslot = (key0 >> 4) * 16u + ((key0 >> 2) & 1u) * 8u + ((key0 >> 3) & 1u) * 4u +
                           (key0 & 3u);
    auto lstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < kKChunks; ++i) {
            const uint32_t e = (uint32_t)i * kThreads + tid;
            *reinterpret_cast<f16x8*>(&kt[buf][(e >> 4) * kKP + 8u * (e & 15u)]) = kr[i];
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            if constexpr (kVKeys == 4) {
                f16x4 w;
                w[0] = vr[0][j];
                w[1] = vr[1][j];
                w[2] = vr[2][j];
                w[3] = vr[3][j];
                *reinterpret_cast<f16x4*>(&vt[buf][(8u * dg + j) * kVP + vslot]) = w;
            } else {
                f16x2 w;
                w[0] = vr[0][j];
                w[1] = vr[1][j];
                *reinterpret_cast<f16x2*>(&vt[buf][(8u * dg + j) * kVP + vslot]) = w;
            }
        }
    };

    // one 64-key tile: S^T = K . Q^T, online softmax, O^T += V^T . P^T
    auto tile_step = [&](int buf, uint32_t j, auto diag_tag) {
        constexpr bool kDiag = decltype(diag_tag)::value;
        f32x16 s[NT][2];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int mt = 0; mt < 2; ++mt) s[nt][mt] = f32x16{};
        // K operands are read one k-step ahead of their MFMAs
        const f16* kbuf = &kt[buf][n * kKP + 8 * hh];
        f16x8 ka[2][2];
        ka[0][0] = lds16(kbuf);
        ka[0][1] = lds16(kbuf + 32 * kKP);
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
            const int cur = ks & 1;
            if (ks + 1 < 8) {
                ka[cur ^ 1][0] = lds16(kbuf + 16 * (ks + 1));
                ka[cur ^ 1][1] = lds16(kbuf + 32 * kKP + 16 * (ks + 1));
            }
#pragma unroll
            for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) s[nt][mt] = mfma32(ka[cur][mt], qb[nt][ks], s[nt][mt]);
        }
        float m_tile[NT];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            float mx = -INFINITY;
#pragma unroll
            for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    float x = s[nt][mt][i];
                    if constexpr (kDiag) {
                        const uint32_t query = q0 + 32u * nt + n;
                        const uint32_t key = j * kBN + 32u * mt + 8u * (i >> 2) + 4u * hh + (i & 3);
                        if (key > query || key >= N) x = -INFINITY;
                        s[nt][mt][i] = x;
                    }
                    mx = fmaxf(mx, x);
                }
            mx = fmaxf(mx, xor_lane(mx, 32));
            m_tile[nt] = mx * a.scale_log2;
        }
        // one (rarely taken) block rescales every column tile, so no part of
        // it is speculated into the common path
        bool need[NT];
        bool any = false;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            need[nt] = m_tile[nt] > m_used[nt] + kRescaleSlack;
            any = any || need[nt];
        }
        if (__any(any)) {
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                const float mn = need[nt] ? m_tile[nt] : m_used[nt];
                const float al = fast_exp2(m_used[nt] - mn);
                l_run[nt] *= al;
#pragma unroll
                for (int dt = 0; dt < 4; ++dt) o[nt][dt] *= al;
                m_used[nt] = mn;
            }
        }
        float mneg[NT], psum[NT];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            mneg[nt] = -m_used[nt];
            psum[nt] = 0.f;
        }
        // P one 16-key MFMA step at a time, consumed at once by that step's
        // PV MFMAs: exps of step ks+1 overlap the MFMAs of step ks
        const f16* vbuf = &vt[buf][n * kVP + 8 * hh];
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            f16x8 va[4];
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) va[dt] = lds16(vbuf + 32 * dt * kVP + 16 * ks);
            f16x8 pb[NT];
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
#pragma unroll
                for (int r = 0; r < 8; ++r)
                    pb[nt][r] = (f16)fast_exp2(__builtin_fmaf(s[nt][ks >> 1][8 * (ks & 1) + r],
                                                              a.scale_log2, mneg[nt]));
                // row sum of the fp16 weights the PV product uses, two per
                // v_dot2_f32_f16 (fp32 accumulate)
#pragma unroll
                for (int r = 0; r < 8; r += 2) {
                    const f16x2 pair = {pb[nt][r], pb[nt][r + 1]};
                    psum[nt] = __builtin_amdgcn_fdot2(pair, f16x2{(f16)1.0f, (f16)1.0f}, psum[nt], false);
                }
            }
#pragma unroll
            for (int dt = 0; dt < 4; ++dt)
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) o[nt][dt] = mfma32(va[dt], pb[nt], o[nt][dt]);
        }
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) l_run[nt] += psum[nt];
    };

    gload(0);
    lstore(0);
    __syncthreads();
    // full tiles 0..tile-1 need no mask; tile `tile` holds the diagonal
    for (uint32_t j = 0; j < tile; ++j) {
        const int buf = (int)(j & 1u);
        gload((j + 1) * kBN);
        tile_step(buf, j, std::false_type{});
        lstore(buf ^ 1);
        __syncthreads();
    }
    tile_step((int)(tile & 1u), tile, std::true_type{});

    // ---- epilogue: O = O^T / l, packed [N][Hq][D]
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        const float l = l_run[nt] + xor_lane(l_run[nt], 32);
        const float inv = 1.f / l;
        const uint32_t query = q0 + 32u * nt + n;
        if (query >= N) continue;
        f16* orow = a.out + ((uint64_t)query * a.num_heads + head) * kD;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
#pragma unroll
            for (int i4 = 0; i4 < 4; ++i4) {
                f16x4 w;
#pragma unroll
                for (int e = 0; e < 4; ++e) w[e] = (f16)(o[nt][dt][4 * i4 + e] * inv);
                *reinterpret_cast<f16x4*>(orow + 32 * dt + 8 * i4 + 4 * hh) = w;
            }
    }
}

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace

int plan_prefill(const PrefillArgs& a) {
    if (get_option(kOptPrefillForceGeneric)) return 0;
    if (a.head_dim != kD) return 0;
    if (a.group == 0 || a.group % 4 != 0 || a.num_heads % 4 != 0) return 0;
    if (a.q_stride % 8 != 0 || a.kv_stride % 8 != 0) return 0;
    if (!aligned16(a.q) || !aligned16(a.k) || !aligned16(a.v) || !aligned16(a.out)) return 0;
    // every row offset must fit the 32-bit buffer ranges
    const uint64_t stride = a.q_stride > a.kv_stride ? a.q_stride : a.kv_stride;
    if ((uint64_t)(a.seq_len + kBM) * stride * 2 + kD * 2 > 0xffffffffull) return 0;
    return 1;
}

hipError_t launch_prefill_kernel(const PrefillArgs& a, int path, hipStream_t stream) {
    if (path != 1) return hipErrorInvalidValue;
    const uint32_t quads = a.num_heads / 4u;
    uint64_t blocks;
    if (quads <= 8 && (8 % quads) == 0) {
        const uint32_t per = 8u / quads;
        blocks = 8ull * ((a.q_tiles + per - 1) / per);
    } else {
        blocks = (uint64_t)a.q_tiles * quads;
    }
    if (blocks > 0x7fffffffull) return hipErrorInvalidValue;
    if (get_option(kOptPrefillWaves) == 4) {
        hipLaunchKernelGGL(prefill_d128<2>, dim3((uint32_t)blocks), dim3(256), 0, stream, a);
    } else {
        hipLaunchKernelGGL(prefill_d128<1>, dim3((uint32_t)blocks), dim3(512), 0, stream, a);
    }
    return hipGetLastError();
}

}  // namespace attn
