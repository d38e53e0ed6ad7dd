// Chunked Flash-Decode for gfx950: single query token, grouped-query heads,
// fp16 KV cache, fp32 softmax, fp16 output.
//
// Reference semantics: causal_attention.hip.cpp:619-716 (per-chunk softmax
// partials) and :719-838 (partial-softmax merge): every key j < kv_len is
// visible; for query head h the KV head is h / (Hq/Hkv); out = softmax(q.K^T /
// sqrt(D)) V in fp32, rounded to fp16.
//
// Design (HBM-bound; 2048*L + 8192 bytes of algorithmic traffic per call):
//  * grid = (nsplit, Hkv).  A workgroup owns one KV head and one contiguous
//    chunk of keys, and serves ALL query heads of the group, so each K/V byte
//    is read from HBM exactly once.
//  * Each wave walks 32-key batches.  Scores come from MFMA
//    v_mfma_f32_16x16x32_f16 as S^T = K . Q^T (keys = rows, the <= 16 grouped
//    query heads = columns): the 16 B K loads are already in A-operand layout.
//    The S^T output leaves lane (gq, n) holding query n and keys 8gq..8gq+7 of
//    the batch (the key rows are permuted so this comes out contiguous), which
//    is exactly the B-operand layout of P^T for the PV product.
//  * PV is O^T = V^T . P^T, also on MFMA.  Lane (gq, n) loads 16 B of V rows
//    8gq..8gq+7 at dims 8n..8n+7 (fully coalesced 256 B rows) and transposes
//    the 8x8 block in registers; MFMA tile mt then covers dims {8n + mt}, so no
//    LDS round trip is needed.  The O^T accumulator of lane (gq, n) ends up
//    holding query n, dims 32gq..32gq+31: no cross-lane reduction of the
//    accumulator, only of the per-query max and sum (two xor shuffles).
//  * The waves of a workgroup merge through LDS.  With nsplit > 1 each
//    workgroup writes an unnormalised partial (max, sum, acc[D]) per query
//    head to the caller's workspace; the last workgroup of a KV head to arrive
//    (an acquire/release arrival counter in the workspace tail, tagged with a
//    per-launch epoch so no initialisation is needed) merges them and writes
//    the fp16 output.  One kernel per decode call, one graph node.
#include "attn_internal.hpp"

#include <algorithm>
#include <atomic>
#include <chrono>

namespace attn {

namespace {

constexpr int kD = 128;
constexpr int kMaxSplits = 256;
constexpr int kAccPitch = kD + 4;

__device__ __forceinline__ bool arrive_last(unsigned long long* ctr, uint32_t epoch,
                                            uint32_t total) {
    unsigned long long old = __hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    unsigned long long nv;
    do {
        nv = ((uint32_t)(old >> 32) == epoch) ? old + 1ull
                                               : (((unsigned long long)epoch << 32) | 1ull);
    } while (!__hip_atomic_compare_exchange_strong(ctr, &old, nv, __ATOMIC_ACQ_REL,
                                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    if ((uint32_t)nv == total) {
        __hip_atomic_store(ctr, ((unsigned long long)epoch << 32), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
        return true;
    }
    return false;
}

template <int WAVES>
__global__ __launch_bounds__(WAVES * 64) void flash_decode_d128(DecodeArgs a) {
    constexpr int kThreads = WAVES * 64;
    // LDS: per-wave (max, sum, acc[16][D]) for the in-workgroup merge; reused
    // for split weights during the cross-workgroup merge.
    __shared__ float s_m[WAVES][16];
    __shared__ float s_l[WAVES][16];
    __shared__ float s_acc[WAVES][16][kAccPitch];
    __shared__ int s_last;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int n = lane & 15;   // MFMA column (query head in group) / A row
    const int gq = lane >> 4;  // MFMA k-group / output row group
    const uint32_t g = blockIdx.y;
    const uint32_t c = blockIdx.x;
    const uint32_t G = a.group;
    const uint32_t t0 = c * a.chunk;
    const uint32_t t1 = min(t0 + a.chunk, a.kv_len);
    const uint32_t last = t1 - 1;
    const uint64_t ks = a.kv_stride;

    // Q^T as the B operand: lane (gq, n) holds Q[g*G + n][32s + 8gq .. +7].
    f16x8 qb[4];
    if ((uint32_t)n < G) {
        const f16* qp = a.q + (uint64_t)(g * G + n) * kD + 8 * gq;
#pragma unroll
        for (int s = 0; s < 4; ++s) qb[s] = ld16(qp + 32 * s);
    } else {
#pragma unroll
        for (int s = 0; s < 4; ++s) qb[s] = f16x8{};
    }

    // S^T row m of tile tt is key 8*(m/4) + 4*tt + (m%4) of the batch, so the
    // output of lane group gq is keys 8gq + (4tt + i).
    const uint32_t krow = 8u * (uint32_t)(n >> 2) + (uint32_t)(n & 3);
    const f16* kb = a.k + (uint64_t)g * kD + 8 * gq;
    const f16* vb = a.v + (uint64_t)g * kD + 8 * n;

    f32x4 acc[8];
#pragma unroll
    for (int mt = 0; mt < 8; ++mt) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY;
    float l_run = 0.f;

    for (uint32_t b0 = t0 + 32u * wave; b0 < t1; b0 += 32u * WAVES) {
        f16x8 kk[2][4];
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            const uint32_t key = min(b0 + krow + 4u * tt, last);
            const f16* p = kb + (uint64_t)key * ks;
#pragma unroll
            for (int s = 0; s < 4; ++s) kk[tt][s] = ld16(p + 32 * s);
        }
        f16x8 vv[8];
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            const uint32_t key = min(b0 + 8u * gq + r, last);
            vv[r] = ld16(vb + (uint64_t)key * ks);
        }
        f32x4 st[2];
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            st[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < 4; ++s)
                st[tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kk[tt][s], qb[s], st[tt], 0, 0, 0);
        }
        // scores of query n for keys b0 + 8gq + r, r = 4tt + i (log2 domain)
        float x[8];
        float mx = -INFINITY;
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t key = b0 + 8u * gq + 4u * tt + i;
                const float v = (key < t1) ? st[tt][i] * a.scale_log2 : -INFINITY;
                x[4 * tt + i] = v;
                mx = fmaxf(mx, v);
            }
        mx = fmaxf(mx, xor_lane(mx, 16));
        mx = fmaxf(mx, xor_lane(mx, 32));
        const float m_new = fmaxf(m_run, mx);
        const float alpha = fast_exp2(m_run - m_new);
        f16x8 pb;
        float psum = 0.f;
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            const f16 p = (f16)fast_exp2(x[r] - m_new);
            pb[r] = p;
            psum += (float)p;
        }
        l_run = l_run * alpha + psum;
        m_run = m_new;
#pragma unroll
        for (int mt = 0; mt < 8; ++mt) {
            acc[mt] *= alpha;
            f16x8 va;
#pragma unroll
            for (int r = 0; r < 8; ++r) va[r] = vv[r][mt];
            acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pb, acc[mt], 0, 0, 0);
        }
    }

    // per-query sum over the four lane groups (the max is already shared)
    l_run += xor_lane(l_run, 16);
    l_run += xor_lane(l_run, 32);
    if (gq == 0) {
        s_m[wave][n] = m_run;
        s_l[wave][n] = l_run;
    }
#pragma unroll
    for (int mt = 0; mt < 8; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) s_acc[wave][n][32 * gq + 8 * i + mt] = acc[mt][i];
    __syncthreads();

    const uint32_t outs = G * kD;
    for (uint32_t idx = tid; idx < outs; idx += kThreads) {
        const uint32_t qn = idx >> 7;
        const uint32_t d = idx & (kD - 1);
        float M = s_m[0][qn];
#pragma unroll
        for (int w = 1; w < WAVES; ++w) M = fmaxf(M, s_m[w][qn]);
        float num = 0.f, den = 0.f;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) {
            const float wt = fast_exp2(s_m[w][qn] - M);
            num += wt * s_acc[w][qn][d];
            den += wt * s_l[w][qn];
        }
        const uint32_t hq = g * G + qn;
        if (a.nsplit == 1) {
            a.out[(uint64_t)hq * kD + d] = (f16)(num / den);
        } else {
            const uint64_t st = (uint64_t)hq * a.nsplit + c;
            a.part_out[st * kD + d] = num;
            if (d == 0) {
                a.part_max[st] = M;
                a.part_sum[st] = den;
            }
        }
    }
    if (a.nsplit == 1) return;

    // ---- cross-workgroup merge by the last arriving workgroup of KV head g
    __threadfence();
    __syncthreads();
    if (tid == 0) s_last = arrive_last(a.counters + g, a.epoch, a.nsplit) ? 1 : 0;
    __syncthreads();
    if (!s_last) return;
    __threadfence();

    const uint32_t S = a.nsplit;
    // weights w[qn][c] = 2^(m_c - M_qn) in the s_acc area (G*S <= 16*512 floats
    // needs 32 KB; s_acc holds WAVES*16*132 floats >= 33 KB for WAVES >= 4)
    float* wts = &s_acc[0][0][0];
    float* Ms = &s_m[0][0];   // [16]
    float* dens = &s_l[0][0]; // [16]
    for (uint32_t idx = tid; idx < G * S; idx += kThreads) {
        const uint32_t qn = idx / S, cc = idx - qn * S;
        wts[idx] = a.part_max[(uint64_t)(g * G + qn) * S + cc];
    }
    __syncthreads();
    // one wave per query head: max and weighted sum
    for (uint32_t qn = wave; qn < G; qn += WAVES) {
        float M = -INFINITY;
        for (uint32_t cc = lane; cc < S; cc += 64) M = fmaxf(M, wts[qn * S + cc]);
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) M = fmaxf(M, xor_lane(M, o));
        float den = 0.f;
        for (uint32_t cc = lane; cc < S; cc += 64) {
            const float w = fast_exp2(wts[qn * S + cc] - M);
            wts[qn * S + cc] = w;
            den += w * a.part_sum[(uint64_t)(g * G + qn) * S + cc];
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) den += xor_lane(den, o);
        if (lane == 0) {
            Ms[qn] = M;
            dens[qn] = den;
        }
    }
    __syncthreads();
    // outputs (qn, 4 dims): the split range is divided among `parts` thread
    // groups, partial sums meet in LDS behind the weights
    const uint32_t items = G * (kD / 4);
    const uint32_t parts = kThreads / items > 0 ? kThreads / items : 1;
    const uint32_t total = items * parts;
    float4* red = reinterpret_cast<float4*>(wts + 16 * kMaxSplits);
    for (uint32_t w = tid; w < total; w += kThreads) {
        const uint32_t item = w % items;
        const uint32_t part = w / items;
        const uint32_t qn = item / (kD / 4);
        const uint32_t d4 = item - qn * (kD / 4);
        const float* po = a.part_out + ((uint64_t)(g * G + qn) * S) * kD + 4 * d4;
        float4 sum = make_float4(0.f, 0.f, 0.f, 0.f);
        for (uint32_t cc = part; cc < S; cc += parts) {
            const float w8 = wts[qn * S + cc];
            const float4 v = *reinterpret_cast<const float4*>(po + (uint64_t)cc * kD);
            sum.x += w8 * v.x;
            sum.y += w8 * v.y;
            sum.z += w8 * v.z;
            sum.w += w8 * v.w;
        }
        red[w] = sum;
    }
    __syncthreads();
    for (uint32_t item = tid; item < items; item += kThreads) {
        float4 t = red[item];
        for (uint32_t p = 1; p < parts; ++p) {
            const float4 u = red[p * items + item];
            t.x += u.x;
            t.y += u.y;
            t.z += u.z;
            t.w += u.w;
        }
        const uint32_t qn = item / (kD / 4);
        const uint32_t d4 = item - qn * (kD / 4);
        const float inv = 1.f / dens[qn];
        // 2-byte stores: `out` only needs fp16 alignment (callers may pass an
        // offset pointer, test_causal_attention.cpp:212)
        f16* o = a.out + (uint64_t)(g * G + qn) * kD + 4 * d4;
        o[0] = (f16)(t.x * inv);
        o[1] = (f16)(t.y * inv);
        o[2] = (f16)(t.z * inv);
        o[3] = (f16)(t.w * inv);
    }
}

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

std::atomic<uint32_t> g_epoch{0};

uint32_t next_epoch() {
    uint32_t e = g_epoch.fetch_add(1, std::memory_order_relaxed);
    if (e == 0) {
        // seed from the clock so a workspace left by another process is very
        // unlikely to carry a matching tag
        const uint32_t seed = (uint32_t)std::chrono::steady_clock::now().time_since_epoch().count();
        uint32_t expected = 1;
        g_epoch.compare_exchange_strong(expected, seed | 1u);
        e = g_epoch.fetch_add(1, std::memory_order_relaxed);
    }
    return e;
}

// LDS needed by the cross-workgroup merge must fit in s_acc: weights
// (16*kMaxSplits floats) + float4 partial sums (at most 16*32*... = max(items,
// threads) float4, items <= 16*32).
static_assert(4 * 16 * kAccPitch >= 16 * kMaxSplits + 4 * 512, "merge scratch exceeds LDS area");

}  // namespace

const void* decode_kernel_symbol(int path) {
    if (path == 1) return reinterpret_cast<const void*>(&flash_decode_d128<4>);
    if (path == 2) return reinterpret_cast<const void*>(&flash_decode_d128<8>);
    return generic_attention_symbol();
}

DecodePlan plan_decode(uint32_t kv_len, uint32_t num_heads, uint32_t num_kv_heads,
                       uint32_t head_dim, uint64_t kv_stride, const void* q, const void* k,
                       const void* v, int device) {
    DecodePlan p{0, 1, kv_len, 256};
    const uint32_t G = num_heads / num_kv_heads;
    const bool mfma_ok = head_dim == kD && G >= 1 && G <= 16 && kv_stride % 8 == 0 &&
                         aligned16(q) && aligned16(k) && aligned16(v) &&
                         get_option(kOptDecodeForceGeneric) == 0;
    if (!mfma_ok) return p;
    const long wopt = get_option(kOptDecodeWaves);
    const int waves = (wopt == 8) ? 8 : 4;
    p.path = (waves == 8) ? 2 : 1;
    p.block = 64u * waves;
    const uint32_t unit = 32u * waves;
    const uint32_t units = (kv_len + unit - 1) / unit;
    const uint32_t cus = (uint32_t)std::max(1, device_cu_count(device));
    long sopt = get_option(kOptDecodeSplits);
    uint32_t target = sopt > 0 ? (uint32_t)sopt : std::max(1u, (2u * cus + num_kv_heads - 1) / num_kv_heads);
    uint32_t nsplit = std::min<uint32_t>({target, units, (uint32_t)kMaxSplits});
    nsplit = std::max(1u, nsplit);
    uint32_t chunk = ((units + nsplit - 1) / nsplit) * unit;
    nsplit = (kv_len + chunk - 1) / chunk;
    // the caller's workspace holds Hq * ceil(L / KV_CHUNK) states
    // (kernels.hpp:103); partials plus the aligned counters must fit.
    const uint64_t cap = (uint64_t)num_heads * ((kv_len + 11u) / 12u);
    while (nsplit > 1 && (uint64_t)num_heads * nsplit + 2ull * num_kv_heads + 2ull > cap) {
        const uint32_t u_per = chunk / unit + 1;
        chunk = u_per * unit;
        nsplit = (kv_len + chunk - 1) / chunk;
    }
    if (nsplit <= 1) {
        nsplit = 1;
        chunk = units * unit;
    }
    p.nsplit = nsplit;
    p.chunk = chunk;
    return p;
}

void replan_decode(DecodeArgs& a, int path, int device) {
    const DecodePlan p = plan_decode(a.kv_len, a.num_heads, a.num_kv_heads, a.head_dim,
                                     a.kv_stride, a.q, a.k, a.v, device);
    (void)path;
    a.nsplit = p.nsplit;
    a.chunk = p.chunk;
    uintptr_t ctr = (uintptr_t)(a.part_sum + (uint64_t)a.num_heads * p.nsplit);
    ctr = (ctr + 7u) & ~(uintptr_t)7u;
    a.counters = reinterpret_cast<unsigned long long*>(ctr);
    a.epoch = next_epoch();
}

hipError_t launch_decode_kernel(const DecodeArgs& a, const DecodePlan& p, hipStream_t stream) {
    if (p.path == 1) {
        hipLaunchKernelGGL(flash_decode_d128<4>, dim3(a.nsplit, a.num_kv_heads), dim3(256), 0,
                           stream, a);
    } else if (p.path == 2) {
        hipLaunchKernelGGL(flash_decode_d128<8>, dim3(a.nsplit, a.num_kv_heads), dim3(512), 0,
                           stream, a);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace attn
