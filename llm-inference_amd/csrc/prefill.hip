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
//    softmax overlaps the other's MFMAs); Q, S and O stay in VGPRs.  Short
//    prompts use 32 query tokens as 4 waves (one per head and SIMD): twice
//    the workgroups, each through its key tiles faster.
//  * K and V of a 64-key tile are staged in LDS once per workgroup and shared
//    by the 4 heads (the reference re-reads them per head), copied straight
//    from global memory into LDS by buffer_load ... lds (no VGPRs, no LDS
//    stores).  K and V rows are unpadded with their 16-byte chunks
//    XOR-swizzled by row, so the MFMA operand reads are free of bank
//    conflicts; a DMA instruction writes 1 KiB of LDS (4 key rows).  Rows
//    past N read as zero through the buffer range check.
//  * S^T = K . Q^T with v_mfma_f32_32x32x16_f16: keys are MFMA rows, queries
//    columns, so each lane holds one query's scores and the online softmax
//    (running max, running sum, rescale) is per lane; the xor-32 exchange
//    with the lane holding the query's other keys is made only when the
//    running maximum moves.  Q is pre-scaled into the exp2 domain and the
//    accumulators start at -m, so the MFMAs return the shifted scores and
//    P = exp2(S) needs no multiply-add per score.
//  * O^T = V^T . P^T on the same MFMA; O^T stays in 64 accumulator registers.
//    The V^T operand comes from row-major V through ds_read_b64_tr_b16 (two
//    4-key transposing reads per operand), with the keys in the order the
//    S^T accumulator produces them, so P never leaves registers.
//  * Causal tile skipping: a workgroup's queries (64, or 32 for the 4-wave
//    variant) visit only the 64-key tiles up to the one holding their last
//    query; that tile, which crosses the diagonal, is masked.  Tiles are handed out longest-first and the
//    four head groups of one KV head are kept on the same pair of XCDs so the
//    KV head's K/V stays in one L2.
//  * Tile j+1 is copied into the other LDS buffer while tile j is computed;
//    one barrier per tile.
//  * Short prompts (N <= 1024) split each 32-query tile's keys over the waves
//    of one head's workgroup and combine the partial states through LDS
//    (prefill_d128<4, true, true>: 64-key tiles over 4 waves, up to 256
//    tokens; prefill_sk32: 32-key units over 8 waves, up to 32 tokens;
//    prefill_skn: 32-key units streamed per wave, from 257 to 1024 tokens).
//    From 1025 to 4096 tokens the 32-query tile of 4 heads is computed by 8
//    waves whose two 4-wave groups split its key tiles (even and odd), with
//    the two states combined through LDS (prefill_d128<8, false, false, true>).
#include "attn_internal.hpp"

#include <type_traits>

namespace attn {

namespace {

constexpr int kD = 128;
constexpr int kBM = 64;        // query tokens per workgroup, at most
constexpr int kBN = 64;        // keys per tile
// K rows are unpadded (256 B) with their 16-byte chunks XOR-swizzled: chunk
// c of row r sits at chunk c ^ (r % 16).  The 16 lanes of one phase of an
// A-operand read (ds_read_b128) address 16 consecutive rows at the same
// chunk, which the swizzle spreads over 16 chunks = the 64 banks; each lane
// keeps one address per k-step (8 VGPRs), so the tile loop gains no
// instruction.  Against 272-byte padded rows it copies 16 KiB per tile
// instead of 17 KiB.
constexpr int kKP = kD;
// V rows are unpadded (256 B) with their 16-byte chunks XOR-swizzled: chunk
// c of row r sits at chunk c ^ 4 (r % 4).  The 32 lanes of half a transposing
// read address 4 consecutive rows (r % 4 = 0..3) x 64 bytes of one 32-dim
// tile; the swizzle puts those rows' 64 bytes in 4 different 64-byte bank
// groups, so they cover the 64 banks once.  Against 320-byte padded rows it
// copies 16 KiB per tile instead of 20 KiB.
constexpr int kVP = kD;
constexpr int kKChunks = kKP / 8;             // 16-byte LDS chunks per K row (16)
constexpr int kVChunks = kVP / 8;             // ... per V row (16)
constexpr int kKDma = kBN * kKChunks / 64;    // 1 KiB DMA instructions per K tile (16)
constexpr int kVDma = kBN * kVChunks / 64;    // ... per V tile (16)
constexpr int kMaxDma = kKDma > kVDma ? kKDma : kVDma;

// s_waitcnt immediate that waits until at most n vector-memory loads are
// outstanding (vmcnt bits 3:0 and 15:14; expcnt and lgkmcnt not waited on)
constexpr int vmcnt_imm(int n) { return 0x0F70 | (n & 0xF) | ((n >> 4) << 14); }
static_assert(vmcnt_imm(0) == 0x0F70 && vmcnt_imm(16) == 0x4F70 && vmcnt_imm(63) == 0xCF7F);

// LDS chunk position pos of K row r holds the row's 16-byte chunk pos ^ (r % 16)
__device__ __forceinline__ uint32_t k_src_chunk(uint32_t r, uint32_t pos) {
    return pos ^ (r & 15u);
}

// LDS offset (halves) of lane (hh, n)'s A operand at k-step ks: row n, the
// 16-byte chunk 2 ks + hh, swizzled
__device__ __forceinline__ uint32_t k_read_offset(uint32_t n, uint32_t hh, uint32_t ks) {
    return n * kKP + 8u * k_src_chunk(n, 2u * ks + hh);
}

// LDS chunk position pos of V row r holds the row's 16-byte chunk pos ^ 4 (r % 4)
__device__ __forceinline__ uint32_t v_src_chunk(uint32_t r, uint32_t pos) {
    return pos ^ (4u * (r & 3u));
}

#define LDS_AS __attribute__((address_space(3)))
typedef short s16x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f16x8 lds16(const f16* p) {
    return *reinterpret_cast<const f16x8*>(p);
}

__device__ __forceinline__ f32x16 mfma32(f16x8 a, f16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// Four fp16 of one LDS column: lane i of each 16-lane group receives element
// i of the 4-element chunks its group addresses, from chunks i/4, 4 + i/4, ...
__device__ __forceinline__ f16x4 lds_tr4(const f16* p) {
    const s16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((LDS_AS s16x4*)(const LDS_AS void*)p);
    return __builtin_bit_cast(f16x4, r);
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

// Key tiles an ALL workgroup stages at once: 4 x (16,384 + 16,384) B of LDS
constexpr uint32_t kAllTiles = 4;

// WAVES = 8: 64 queries of 4 heads per workgroup, two waves per SIMD (long
// prompts); WAVES = 4: 32 queries of 4 heads, one wave per SIMD, so a short
// prompt's few workgroups each finish their chain of key tiles sooner.
// ALL (WAVES = 4, at most kAllTiles key tiles, i.e. N <= 256): every key tile
// the workgroup needs is copied into LDS at once and awaited once, instead of
// one tile ahead of the compute.  A short prompt's chain of tiles is
// otherwise bound by the copy latency, not by the compute: per-wave
// timestamps at N = 254 showed ~1.9 us per tile (the next tile's copy,
// issued at the start of a tile, completing after the tile's compute)
// against ~0.8 us per tile once the copies hit L2 at N = 1024.
// SK (with ALL): the key tiles of one query tile are split over the waves.
// A workgroup is ONE head's 32-query tile; wave w copies and computes key
// tile w (if it exists) with its own softmax state, and the states are
// combined through LDS (M = max(m_a, m_b); l and O scaled by 2^(m - M) and
// added), so the chain of up to 4 dependent tiles becomes one tile plus the
// combine, and a short prompt gets 4x the workgroups (one per head instead
// of per 4 heads): C2 (254 tokens) 10.1 -> 6.6 us, 64 tokens 6.3 -> 4.7 us.
// KS2 (WAVES = 8, streaming): a workgroup is a 32-query tile of 4 heads; wave
// w computes head w % 4, and the group w / 4 takes the even or the odd key
// tiles with its own softmax state, two tiles staged per step; the second
// group's state is folded into the first's through LDS at the end.
template <int WAVES, bool ALL, bool SK, bool KS2 = false>
__global__ __launch_bounds__(64 * WAVES, 1) void prefill_d128(PrefillArgs a) {
    static_assert(!ALL || WAVES == 4, "the all-tiles variant is the 4-wave kernel");
    static_assert(!SK || ALL, "split keys needs every key tile staged at once");
    static_assert(!KS2 || (WAVES == 8 && !ALL), "key halves: the 8-wave streaming tile");
    constexpr int kW = WAVES;
    // query tokens per workgroup (KS2: 32 queries, the two 4-wave groups
    // split the key tiles)
    constexpr int kBMw = KS2 ? 32 : 8 * WAVES;
    constexpr int kDpw = (kMaxDma + WAVES - 1) / WAVES;   // DMA instructions per wave
    // two LDS buffers per operand as distinct objects, so the compiler can
    // tell a DMA into one buffer from the reads of the other (ALL: one buffer
    // per key tile, all filled before any is read; KS2: two key tiles per
    // buffer, one per group)
    constexpr int kTiles = ALL ? (int)kAllTiles : (KS2 ? 2 : 1);
    constexpr int kKBuf = kTiles * kBN * kKP;
    constexpr int kVBuf = kTiles * kBN * kVP;
    __shared__ __attribute__((aligned(16))) f16 kt0[kKBuf];
    __shared__ __attribute__((aligned(16))) f16 kt1[ALL ? 8 : kKBuf];
    __shared__ __attribute__((aligned(16))) f16 vt0[kVBuf];
    __shared__ __attribute__((aligned(16))) f16 vt1[ALL ? 8 : kVBuf];
    // split keys: each wave's (m, l) for the combine (KS2: the second group's)
    __shared__ f32x2 sml[SK ? kAllTiles : (KS2 ? 4 : 1)][64];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: SGPR descriptors
    const int n = lane & 31;   // MFMA column (query) / A-operand row
    const int hh = lane >> 5;  // MFMA k-half / output row half

    uint32_t tile, head, g, q0;  // q0: this wave's first query
    if constexpr (SK) {
        if (!map_block(blockIdx.x, a.num_heads, a.q_tiles, head, tile)) return;
        g = head / a.group;
        q0 = tile * kBMw;
    } else {
        const uint32_t quads = a.num_heads / 4u;
        uint32_t quad;
        if (!map_block(blockIdx.x, quads, a.q_tiles, quad, tile)) return;
        head = 4u * quad + (uint32_t)(wave & 3);
        g = (4u * quad) / a.group;
        q0 = tile * kBMw + (KS2 ? 0u : 32u * (uint32_t)(wave >> 2));
    }
    // the query tile's last key tile, which holds its diagonal
    const uint32_t last = (tile * kBMw + kBMw - 1) / kBN;
    const uint32_t N = a.seq_len;
    const uint32_t q_row_bytes = (uint32_t)(a.q_stride * 2);
    const uint32_t kv_row_bytes = (uint32_t)(a.kv_stride * 2);

    // Q^T B operands: lane (hh, n) holds Q[q0 + n][head][16s + 8hh .. +7] for
    // k-step s; rows past N read as zero
    const BufRsrc rq = make_rsrc(a.q + (uint64_t)head * kD,
                                 __builtin_amdgcn_readfirstlane((N - 1) * q_row_bytes + kD * 2));
    f16x8 qb[8];
    {
        const uint32_t off = (q0 + n) * q_row_bytes + 16u * hh;
#pragma unroll
        for (int s = 0; s < 8; ++s) qb[s] = buf_ld16(rq, off + 32u * s);
    }

    f32x16 o[4];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) o[dt] = f32x16{};
    float m_used = -INFINITY, l_run = 0.f;
    // kShift: scores leave the QK MFMAs in exp2 units and already shifted.
    // Q is scaled by log2(e)/sqrt(D) once (rounded to fp16) and each tile's
    // accumulators start at -m_cur (negm, 16 copies) instead of 0, so
    // P = exp2(s) takes no per-score multiply-add (32 v_fma_f32 per wave and
    // tile): C4 264.8 -> 256.9 us, 4096 tokens 94.5 -> 91.7 us.  m_cur is 0
    // until the first rescale sets it to m_used; thr = m_used + slack - m_cur.
    // The split-keys form (one tile per wave) keeps the multiply-add: there
    // the one-time scaling of Q sits on the critical path (C2 +0.3 us).
    constexpr bool kShift = !SK;
    f32x16 negm = f32x16{};
    float m_cur = 0.f, thr = -INFINITY;
    auto scale_q = [&]() {
        if constexpr (kShift) {
#pragma unroll
            for (int s = 0; s < 8; ++s)
#pragma unroll
                for (int e = 0; e < 8; ++e) qb[s][e] = (f16)((float)qb[s][e] * a.scale_log2);
        }
    };

    // LDS-DMA staging.  DMA instruction i of a tile fills LDS bytes
    // [1024 i, 1024 i + 1024) of the buffer; lane L writes 16-byte chunk
    // q = 64 i + L = row * chunks + c, fetched from key row `row`, bytes 16c
    // (c past the row's 16 data chunks is padding: bytes 0..15 again).  Wave w
    // issues instructions w, w + WAVES, w + 2 WAVES, ...
    uint32_t koff[kDpw], voff[kDpw];
#pragma unroll
    for (int t = 0; t < kDpw; ++t) {
        const uint32_t q = (uint32_t)(wave + kW * t) * 64u + (uint32_t)lane;
        const uint32_t kr = q / kKChunks, kc = q % kKChunks;
        const uint32_t vr = q / kVChunks, vc = q % kVChunks;
        koff[t] = kr * kv_row_bytes + k_src_chunk(kr, kc) * 16u;
        voff[t] = vr * kv_row_bytes + v_src_chunk(vr, vc) * 16u;
    }
    const f16* kbase = a.k + (uint64_t)g * kD;
    const f16* vbase = a.v + (uint64_t)g * kD;
    auto stage = [&](uint32_t kv0, f16* kt, f16* vt) {
        // resources start at row kv0 and end at row N - 1
        const uint32_t rows = N > kv0 ? N - kv0 : 0u;
        const uint32_t bytes =
            __builtin_amdgcn_readfirstlane(rows ? (rows - 1u) * kv_row_bytes + kD * 2 : 0u);
        const BufRsrc rk = make_rsrc(kbase + (uint64_t)kv0 * a.kv_stride, bytes);
        const BufRsrc rv = make_rsrc(vbase + (uint64_t)kv0 * a.kv_stride, bytes);
#pragma unroll
        for (int t = 0; t < kDpw; ++t) {
            const int i = wave + kW * t;
            if (i < kKDma)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    rk, (LDS_AS void*)((LDS_AS char*)(LDS_AS void*)kt + 1024 * i), 16,
                    (int)koff[t], 0, 0, 0);
            if (i < kVDma)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    rv, (LDS_AS void*)((LDS_AS char*)(LDS_AS void*)vt + 1024 * i), 16,
                    (int)voff[t], 0, 0, 0);
        }
    };
    // the DMA writes become visible to the workgroup after the vmcnt wait and
    // the barrier that follows it
    auto publish = [&]() {
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
        __syncthreads();
    };

    // transposing-read address of lane (hh, n): group grp = lane / 16 holds
    // dims 16 (grp & 1) + 0..15 of a 32-dim tile; its lane j addresses key
    // 4 hh + j / 4 (+ the k-step and half offsets, multiples of 8 keys, so
    // the key's r % 4 is j / 4), dims 4 (j & 3) + 0..3, whose chunk of dim
    // tile dt is swizzled to 4 (dt ^ (j / 4)) + 2 (grp & 1) + (j & 3) / 2
    const uint32_t grp = (uint32_t)lane >> 4, jl = (uint32_t)lane & 15u;
    const uint32_t vrd = (4u * hh + (jl >> 2)) * kVP + 16u * (grp & 1u) + 4u * (jl & 3u);
    uint32_t vdt[4];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) vdt[dt] = vrd + 32u * ((uint32_t)dt ^ (jl >> 2));
    uint32_t kofs[8];
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) kofs[ks] = k_read_offset(n, hh, ks);

    // one 64-key tile: S^T = K . Q^T, online softmax, O^T += V^T . P^T
    // kVWait: the caller's V copy may still be in flight (split keys: the K
    // copy was issued first and awaited alone), so wait for it before PV
    auto tile_step = [&](const f16* kt, const f16* vt, uint32_t j, auto diag_tag,
                         auto v_wait_tag) {
        constexpr bool kDiag = decltype(diag_tag)::value;
        constexpr bool kVWait = decltype(v_wait_tag)::value;
        // the compiler's interleaving strategy for LDS reads and MFMAs
        // (iglp_opt 0), identical bits: 8-wave tile at C4 261.7 against
        // 265.8 us (median of six 100-launch medians each, same box); 4-wave
        // tile at 2048 tokens 39.0 against 41.4 us, 3072 61.6 against 63.4
        // us; the all-tiles-staged forms of short prompts are level or slower
        // with it (254 tokens 8.2 against 8.1 us)
        if constexpr (!ALL) __builtin_amdgcn_iglp_opt(0);
        f32x16 s[2] = {negm, negm};
        // K operands are read one k-step ahead of their MFMAs (rows n and
        // n + 32 share the swizzle)
        f16x8 ka[2][2];
        ka[0][0] = lds16(kt + kofs[0]);
        ka[0][1] = lds16(kt + kofs[0] + 32 * kKP);
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
            const int cur = ks & 1;
            if (ks + 1 < 8) {
                ka[cur ^ 1][0] = lds16(kt + kofs[ks + 1]);
                ka[cur ^ 1][1] = lds16(kt + kofs[ks + 1] + 32 * kKP);
            }
#pragma unroll
            for (int mt = 0; mt < 2; ++mt) s[mt] = mfma32(ka[cur][mt], qb[ks], s[mt]);
        }
        float mx = -INFINITY;
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                float x = s[mt][i];
                if constexpr (kDiag) {
                    const uint32_t query = q0 + n;
                    const uint32_t key = j * kBN + 32u * mt + 8u * (i >> 2) + 4u * hh + (i & 3);
                    if (key > query || key >= N) x = -INFINITY;
                    s[mt][i] = x;
                }
                mx = fmaxf(mx, x);
            }
        // lanes n and n + 32 hold one query's keys and share m_used; the
        // pair's maximum exceeds m_used + slack iff one lane's own maximum
        // does, so the exchange of the two (a lane swap) is only made
        // in the rescale block.  One (rarely taken) block rescales, so none of
        // it is speculated into the common path.  The scores are relative to
        // m_cur: the block moves them, m_cur and negm to the new m_used.
        if constexpr (kShift) {
            if (__any(mx > thr)) {
                const float m_tile = max_xor<32>(mx) + m_cur;
                const float mn = (m_tile > m_used + kRescaleSlack) ? m_tile : m_used;
                const float al = fast_exp2(m_used - mn);
                l_run *= al;
#pragma unroll
                for (int dt = 0; dt < 4; ++dt) o[dt] *= al;
                m_used = mn;
                const float d = mn - m_cur;
#pragma unroll
                for (int mt = 0; mt < 2; ++mt) s[mt] -= d;
                m_cur = mn;
                negm = -mn;
                thr = kRescaleSlack;
            }
        } else {
            const float m_lane = mx * a.scale_log2;
            if (__any(m_lane > m_used + kRescaleSlack)) {
                const float m_tile = max_xor<32>(m_lane);
                const float mn = (m_tile > m_used + kRescaleSlack) ? m_tile : m_used;
                const float al = fast_exp2(m_used - mn);
                l_run *= al;
#pragma unroll
                for (int dt = 0; dt < 4; ++dt) o[dt] *= al;
                m_used = mn;
            }
        }
        const float mneg = -m_used;
        float psum = 0.f;

        // P one 16-key MFMA step at a time, consumed at once by that step's
        // PV MFMAs: exps of step ks+1 overlap the MFMAs of step ks.  Step ks
        // covers keys 32 (ks / 2) + 16 (ks % 2) + 8 (e / 4) + 4 hh + e % 4.
        if constexpr (kVWait) __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const int koffs = (32 * (ks >> 1) + 16 * (ks & 1)) * kVP;
            f16x8 va[4];
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) {
                const f16x4 lo = lds_tr4(vt + vdt[dt] + koffs);
                const f16x4 hi = lds_tr4(vt + vdt[dt] + koffs + 8 * kVP);
                va[dt] = f16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            }
            f16x8 pb;
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                const float x = s[ks >> 1][8 * (ks & 1) + r];
                if constexpr (kShift) pb[r] = (f16)fast_exp2(x);
                else pb[r] = (f16)fast_exp2(__builtin_fmaf(x, a.scale_log2, mneg));
            }
            // row sum of the fp16 weights the PV product uses, two per
            // v_dot2_f32_f16 (fp32 accumulate)
#pragma unroll
            for (int r = 0; r < 8; r += 2) {
                const f16x2 pair = {pb[r], pb[r + 1]};
                psum = __builtin_amdgcn_fdot2(pair, f16x2{(f16)1.0f, (f16)1.0f}, psum, false);
            }
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) o[dt] = mfma32(va[dt], pb, o[dt]);
        }
        l_run += psum;
    };

    if constexpr (SK) {
        // wave t copies and computes key tile t alone: its own DMA, its own
        // wait (a wave sees its LDS-DMA writes once vmcnt reaches 0), no
        // workgroup barrier before the compute
        const uint32_t t = (uint32_t)wave;
        f16* ktt = kt0 + t * (kBN * kKP);
        f16* vtt = vt0 + t * (kBN * kVP);
        if (t <= last) {
            const uint32_t kv0 = t * kBN;
            const uint32_t rows = N > kv0 ? N - kv0 : 0u;
            const uint32_t bytes =
                __builtin_amdgcn_readfirstlane(rows ? (rows - 1u) * kv_row_bytes + kD * 2 : 0u);
            const BufRsrc rk = make_rsrc(kbase + (uint64_t)kv0 * a.kv_stride, bytes);
            const BufRsrc rv = make_rsrc(vbase + (uint64_t)kv0 * a.kv_stride, bytes);
#pragma unroll
            for (int i = 0; i < kKDma; ++i) {
                const uint32_t q = (uint32_t)i * 64u + (uint32_t)lane;
                const uint32_t kr = q / kKChunks, kc = q % kKChunks;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    rk, (LDS_AS void*)((LDS_AS char*)(LDS_AS void*)ktt + 1024 * i), 16,
                    (int)(kr * kv_row_bytes + k_src_chunk(kr, kc) * 16u), 0, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < kVDma; ++i) {
                const uint32_t q = (uint32_t)i * 64u + (uint32_t)lane;
                const uint32_t vr = q / kVChunks, vc = q % kVChunks;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    rv, (LDS_AS void*)((LDS_AS char*)(LDS_AS void*)vtt + 1024 * i), 16,
                    (int)(vr * kv_row_bytes + v_src_chunk(vr, vc) * 16u), 0, 0, 0);
            }
            // Q and K have landed once at most the kVDma V copies are
            // outstanding (loads complete in order); V is awaited before PV
            __builtin_amdgcn_s_waitcnt(vmcnt_imm(kVDma));
            scale_q();
            if (t < last)
                tile_step(ktt, vtt, t, std::false_type{}, std::true_type{});
            else
                tile_step(ktt, vtt, t, std::true_type{}, std::true_type{});
        }
        if (last == 0) {
            // one tile: wave 0 holds the whole state and finishes below
            if (wave != 0) return;
        } else {
            // Every wave with a tile has a finite m_used: full tiles hold only
            // keys below the first query (and below N), and the diagonal tile
            // holds key 64 last <= every query of the tile.  The waves with a
            // tile leave (O^T, m, l) in LDS over their own K tile, which no
            // other wave reads, so no barrier precedes the writes (C2 6.64 ->
            // 6.53 us); then wave w folds the 32 output dims 32 w .. 32 w + 31
            // of every state and stores them, so the epilogue's work is split
            // four ways.  Keeping wave w's own words in registers instead of
            // reading them back measured slower (6.7-6.8 us).
            // State of wave t in LDS, 16-byte words per lane: [t][16][64] x
            // f32x4 = 16,384 B per wave = one K tile (word e: O^T dims of
            // o[e / 4][4 (e % 4) .. +3]), and (m, l) in sml[t][lane]
            f32x4* st = reinterpret_cast<f32x4*>(kt0);  // [4][16][64] (65,536 B)
            if (t <= last) {
                f32x4* w = st + t * (16u * 64u) + (uint32_t)lane;
#pragma unroll
                for (int e = 0; e < 16; ++e)
                    w[64 * e] = f32x4{o[e >> 2][4 * (e & 3)], o[e >> 2][4 * (e & 3) + 1],
                                      o[e >> 2][4 * (e & 3) + 2], o[e >> 2][4 * (e & 3) + 3]};
                sml[t][lane] = f32x2{m_used, l_run};
            }
            __syncthreads();
            const int dt = wave;
            float m = -INFINITY, l = 0.f;
            f32x16 acc = f32x16{};
            for (uint32_t w2 = 0; w2 <= last; ++w2) {
                const f32x4* w = st + w2 * (16u * 64u) + (uint32_t)lane;
                const f32x2 ml = sml[w2][lane];
                f32x4 ow[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) ow[q] = w[64 * (4 * dt + q)];
                const float mx = fmaxf(m, ml[0]);  // finite: ml[0] is
                const float a1 = fast_exp2(m - mx), a2 = fast_exp2(ml[0] - mx);
                l = l * a1 + ml[1] * a2;
#pragma unroll
                for (int i = 0; i < 16; ++i) acc[i] = acc[i] * a1 + ow[i >> 2][i & 3] * a2;
                m = mx;
            }
            const float inv = 1.f / add_xor<32>(l);
            const uint32_t query = q0 + n;
            if (query < N) {
                f16* orow = a.out + ((uint64_t)query * a.num_heads + head) * kD;
#pragma unroll
                for (int i4 = 0; i4 < 4; ++i4) {
                    f16x4 w;
#pragma unroll
                    for (int e = 0; e < 4; ++e) w[e] = (f16)(acc[4 * i4 + e] * inv);
                    *reinterpret_cast<f16x4*>(orow + 32 * dt + 8 * i4 + 4 * hh) = w;
                }
            }
            return;
        }
    } else if constexpr (KS2) {
        // Key tiles split over the two 4-wave groups: group gk = wave / 4
        // computes tiles gk, gk + 2, gk + 4, ... of the workgroup's 32-query
        // tile with its own softmax state.  Step s stages tiles 2s and 2s + 1
        // side by side into buffer s & 1 (one barrier per step), so a query
        // tile's chain of steps is half its chain of key tiles.
        const uint32_t gk = (uint32_t)wave >> 2;
        const uint32_t steps = (last + 2u) / 2u;
        auto stage2 = [&](uint32_t st, f16* kt, f16* vt) {
            stage(2u * st * kBN, kt, vt);
            if (2u * st + 1u <= last) stage((2u * st + 1u) * kBN, kt + kBN * kKP, vt + kBN * kVP);
        };
        // steps before the last hold two full tiles
        auto full = [&](uint32_t st, const f16* kt, const f16* vt) {
            tile_step(kt + gk * (kBN * kKP), vt + gk * (kBN * kVP), 2u * st + gk,
                      std::false_type{}, std::false_type{});
        };
        // the last step holds tile `last` (the diagonal) and, when `last` is
        // odd, the full tile last - 1
        auto final_step = [&](uint32_t st, const f16* kt, const f16* vt) {
            const uint32_t j = 2u * st + gk;
            if (j == last)
                tile_step(kt + gk * (kBN * kKP), vt + gk * (kBN * kVP), j, std::true_type{},
                          std::false_type{});
            else if (j < last)
                tile_step(kt + gk * (kBN * kKP), vt + gk * (kBN * kVP), j, std::false_type{},
                          std::false_type{});
        };
        stage2(0, kt0, vt0);
        publish();
        scale_q();
        uint32_t st = 0;
        for (; st + 2 < steps; st += 2) {
            stage2(st + 1, kt1, vt1);
            full(st, kt0, vt0);
            publish();
            stage2(st + 2, kt0, vt0);
            full(st + 1, kt1, vt1);
            publish();
        }
        if (st + 1 < steps) {
            stage2(st + 1, kt1, vt1);
            full(st, kt0, vt0);
            publish();
            final_step(st + 1, kt1, vt1);
        } else {
            final_step(st, kt0, vt0);
        }
        // The second group hands (O^T, m, l) of its head to the first through
        // LDS (16 KiB per head: heads 0-1 over the K buffer 0, 2-3 over the V
        // buffer 0, once every wave is past its last tile's reads), and the
        // first group folds it in: M = max(m_a, m_b), l and O^T scaled by
        // 2^(m - M) and added.  A group without a tile (one-tile query tiles)
        // holds m = -inf, l = 0, O = 0 and adds nothing.
        const uint32_t hw = (uint32_t)wave & 3u;
        __syncthreads();
        if (gk == 1) {
            auto put = [&](f16* base) {
                f32x4* w = reinterpret_cast<f32x4*>(base) + (hw & 1u) * 1024u + (uint32_t)lane;
#pragma unroll
                for (int e = 0; e < 16; ++e)
                    w[64 * e] = f32x4{o[e >> 2][4 * (e & 3)], o[e >> 2][4 * (e & 3) + 1],
                                      o[e >> 2][4 * (e & 3) + 2], o[e >> 2][4 * (e & 3) + 3]};
            };
            if (hw < 2) put(kt0);
            else put(vt0);
            sml[hw][lane] = f32x2{m_used, l_run};
        }
        __syncthreads();
        if (gk == 1) return;
        {
            const f32x2 ml = sml[hw][lane];
            const float mm = fmaxf(m_used, ml[0]);  // m_used is finite: tile 0 is this group's
            const float a1 = fast_exp2(m_used - mm), a2 = fast_exp2(ml[0] - mm);
            l_run = l_run * a1 + ml[1] * a2;
            auto fold = [&](const f16* base) {
                const f32x4* w =
                    reinterpret_cast<const f32x4*>(base) + (hw & 1u) * 1024u + (uint32_t)lane;
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const f32x4 x = w[64 * e];
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        o[e >> 2][4 * (e & 3) + i] = o[e >> 2][4 * (e & 3) + i] * a1 + x[i] * a2;
                }
            };
            if (hw < 2) fold(kt0);
            else fold(vt0);
            m_used = mm;
        }
    } else if constexpr (ALL) {
        // tiles 0..last (last < kAllTiles) side by side, one wait
        for (uint32_t t = 0; t <= last; ++t)
            stage(t * kBN, kt0 + t * (kBN * kKP), vt0 + t * (kBN * kVP));
        publish();
        scale_q();
        {
#pragma unroll 1
            for (uint32_t t = 0; t < last; ++t)
                tile_step(kt0 + t * (kBN * kKP), vt0 + t * (kBN * kVP), t, std::false_type{}, std::false_type{});
            tile_step(kt0 + last * (kBN * kKP), vt0 + last * (kBN * kVP), last, std::true_type{}, std::false_type{});
        }
    } else {
    // Tile t sits in buffer t & 1.  Full tiles 0..last-1 need no mask; tile
    // `last` holds the diagonal.  The DMA of tile j+1 goes into the buffer
    // last read before the previous barrier.
    stage(0, kt0, vt0);
    publish();
    scale_q();
    uint32_t j = 0;
    for (; j + 2 <= last; j += 2) {
        stage((j + 1) * kBN, kt1, vt1);
        tile_step(kt0, vt0, j, std::false_type{}, std::false_type{});
        publish();
        stage((j + 2) * kBN, kt0, vt0);
        tile_step(kt1, vt1, j + 1, std::false_type{}, std::false_type{});
        publish();
    }
    if (j < last) {  // j even: tile j in buffer 0, the diagonal tile j + 1 in buffer 1
        stage((j + 1) * kBN, kt1, vt1);
        tile_step(kt0, vt0, j, std::false_type{}, std::false_type{});
        publish();
        tile_step(kt1, vt1, last, std::true_type{}, std::false_type{});
    } else {
        tile_step(kt0, vt0, last, std::true_type{}, std::false_type{});
    }
    }

    // ---- epilogue: O = O^T / l, packed [N][Hq][D]
    const float l = add_xor<32>(l_run);
    const float inv = 1.f / l;
    const uint32_t query = q0 + n;
    if (query < N) {
        f16* orow = a.out + ((uint64_t)query * a.num_heads + head) * kD;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
#pragma unroll
            for (int i4 = 0; i4 < 4; ++i4) {
                f16x4 w;
#pragma unroll
                for (int e = 0; e < 4; ++e) w[e] = (f16)(o[dt][4 * i4 + e] * inv);
                *reinterpret_cast<f16x4*>(orow + 32 * dt + 8 * i4 + 4 * hh) = w;
            }
    }
}

// Split keys over 8 waves of 32 keys each (N <= 256).  A workgroup is ONE
// head's 32-query tile (queries 32 t .. 32 t + 31, keys 0 .. 32 t + 31); wave
// w owns key unit w (keys 32 w .. 32 w + 31) if w <= t.  Each wave copies its
// K unit and V unit (32 swizzled rows each: 8 DMA instructions each) into its
// own 16 KiB LDS region, waits for its own copy, and
// computes S^T, the exact maximum of its 32 keys (one unit per wave, so no
// running rescale), P and O^T.  Its state (O^T) then overwrites its own
// region and (m, l) goes to a small array; after one barrier wave w folds output dims 32 (w / 2) + 8 i4 +
// 4 hh + 0..3 for i4 = 2 (w % 2), 2 (w % 2) + 1 over the states
// (M = max m, l and O scaled by 2^(m - M) and added) and stores them.
// Against the 4-wave form (one 64-key tile per wave): half the copy and half
// the dependent MFMA chain per wave on the critical path, two waves per SIMD,
// but twice the states to combine (16 KiB of fp32 O^T per unit, written
// and read back through LDS).
constexpr int kSkUnit = 32;                            // keys per wave
constexpr int kSkWaves = 8;                            // units per query tile, at most
constexpr int kSkKDma = kSkUnit * kKChunks / 64;       // 8
constexpr int kSkVDma = kSkUnit * kVChunks / 64;       // 8
constexpr int kSkRegion = (kSkKDma + kSkVDma) * 1024;  // 16,384 B per wave
constexpr uint32_t kSkMaxTokens = kSkWaves * kSkUnit;  // 256

__global__ __launch_bounds__(64 * kSkWaves, 1) void prefill_sk32(PrefillArgs a) {
    __shared__ __attribute__((aligned(16))) char lds[kSkWaves * kSkRegion];
    __shared__ f32x2 sml[kSkWaves][64];  // each unit's (m, l)
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n = lane & 31;
    const int hh = lane >> 5;
    uint32_t head, tile;
    if (!map_block(blockIdx.x, a.num_heads, a.q_tiles, head, tile)) return;
    const uint32_t last = tile;  // the query tile's diagonal unit
    // one unit: wave 0 holds the whole state and finishes it alone
    if (last == 0 && wave != 0) return;
    const uint32_t u = (uint32_t)wave;
    const uint32_t g = head / a.group;
    const uint32_t q0 = tile * (uint32_t)kSkUnit;
    const uint32_t N = a.seq_len;
    const uint32_t kv_row_bytes = (uint32_t)(a.kv_stride * 2);
    char* region = lds + u * kSkRegion;

    f32x16 o[4];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) o[dt] = f32x16{};
    float m_unit = -INFINITY, l_unit = 0.f;
    if (u <= last) {
        // the unit's rows start at kv0 < N (kv0 <= q0 and tile t exists only
        // if q0 < N); rows past N read as zero
        const uint32_t kv0 = u * (uint32_t)kSkUnit;
        const uint32_t bytes = __builtin_amdgcn_readfirstlane((N - kv0 - 1u) * kv_row_bytes + kD * 2);
        const BufRsrc rk = make_rsrc(a.k + (uint64_t)kv0 * a.kv_stride + (uint64_t)g * kD, bytes);
        const BufRsrc rv = make_rsrc(a.v + (uint64_t)kv0 * a.kv_stride + (uint64_t)g * kD, bytes);
#pragma unroll
        for (int i = 0; i < kSkKDma; ++i) {
            const uint32_t q = (uint32_t)i * 64u + (uint32_t)lane;
            const uint32_t kr = q / kKChunks, kc = q % kKChunks;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rk, (LDS_AS void*)((LDS_AS char*)(LDS_AS void*)region + 1024 * i), 16,
                (int)(kr * kv_row_bytes + k_src_chunk(kr, kc) * 16u), 0, 0, 0);
        }
        // Q^T B operands (lane (hh, n): Q[q0 + n][head][16 s + 8 hh .. +7]),
        // loaded between the K and the V copies; rows past N read as zero
        const uint32_t q_row_bytes = (uint32_t)(a.q_stride * 2);
        const BufRsrc rq = make_rsrc(a.q + (uint64_t)head * kD,
                                     __builtin_amdgcn_readfirstlane((N - 1) * q_row_bytes + kD * 2));
        f16x8 qb[8];
        const uint32_t qoff = (q0 + n) * q_row_bytes + 16u * hh;
#pragma unroll
        for (int s = 0; s < 8; ++s) qb[s] = buf_ld16(rq, qoff + 32u * s);
#pragma unroll
        for (int i = 0; i < kSkVDma; ++i) {
            const uint32_t q = (uint32_t)i * 64u + (uint32_t)lane;
            const uint32_t vr = q / kVChunks, vc = q % kVChunks;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rv, (LDS_AS void*)((LDS_AS char*)(LDS_AS void*)region + 1024 * (kSkKDma + i)), 16,
                (int)(vr * kv_row_bytes + v_src_chunk(vr, vc) * 16u), 0, 0, 0);
        }
        // a wave sees its own LDS-DMA writes once they are no longer counted
        // in vmcnt (loads complete in order): K and Q have landed once at
        // most the kSkVDma V copies are outstanding; V is awaited before PV
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(kSkVDma));

        const f16* kt = reinterpret_cast<const f16*>(region);
        const f16* vt = reinterpret_cast<const f16*>(region + kSkKDma * 1024);
        // S^T = K . Q^T: lane (hh, n) holds keys 8 (i / 4) + 4 hh + i % 4 of
        // the unit for query n
        f32x16 s = f32x16{};
#pragma unroll
        for (int ks = 0; ks < 8; ++ks)
            s = mfma32(lds16(kt + k_read_offset((uint32_t)n, (uint32_t)hh, (uint32_t)ks)), qb[ks], s);
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            float x = s[i];
            if (u == last) {
                // the diagonal unit starts at q0: mask keys past the query and past N
                const uint32_t key = q0 + 8u * (uint32_t)(i >> 2) + 4u * hh + (uint32_t)(i & 3);
                if (key > q0 + n || key >= N) x = -INFINITY;
                s[i] = x;
            }
            mx = fmaxf(mx, x);
        }
        // finite: key kv0 <= q0 <= every query of the tile, and kv0 < N
        mx = max_xor<32>(mx);
        m_unit = mx * a.scale_log2;
        const float mneg = -m_unit;
        const uint32_t grp = (uint32_t)lane >> 4, jl = (uint32_t)lane & 15u;
        const f16* vb = vt + (4u * hh + (jl >> 2)) * kVP + 16u * (grp & 1u) + 4u * (jl & 3u);
        uint32_t vdt[4];
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) vdt[dt] = 32u * ((uint32_t)dt ^ (jl >> 2));
        float psum = 0.f;
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            f16x8 va[4];
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) {
                const f16x4 lo = lds_tr4(vb + vdt[dt] + 16 * ks * kVP);
                const f16x4 hi = lds_tr4(vb + vdt[dt] + (16 * ks + 8) * kVP);
                va[dt] = f16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            }
            f16x8 pb;
#pragma unroll
            for (int r = 0; r < 8; ++r)
                pb[r] = (f16)fast_exp2(__builtin_fmaf(s[8 * ks + r], a.scale_log2, mneg));
#pragma unroll
            for (int r = 0; r < 8; r += 2) {
                const f16x2 pair = {pb[r], pb[r + 1]};
                psum = __builtin_amdgcn_fdot2(pair, f16x2{(f16)1.0f, (f16)1.0f}, psum, false);
            }
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) o[dt] = mfma32(va[dt], pb, o[dt]);
        }
        l_unit = psum;
    }
    const uint32_t query = q0 + n;
    if (last == 0) {
        const float inv = 1.f / add_xor<32>(l_unit);
        if (query < N) {
            f16* orow = a.out + ((uint64_t)query * a.num_heads + head) * kD;
#pragma unroll
            for (int dt = 0; dt < 4; ++dt)
#pragma unroll
                for (int i4 = 0; i4 < 4; ++i4) {
                    f16x4 w;
#pragma unroll
                    for (int e = 0; e < 4; ++e) w[e] = (f16)(o[dt][4 * i4 + e] * inv);
                    *reinterpret_cast<f16x4*>(orow + 32 * dt + 8 * i4 + 4 * hh) = w;
                }
        }
        return;
    }
    // state of unit u over its own region, 16-byte words per lane: words
    // 0-15 O^T (word e = o[e / 4][4 (e % 4) .. +3]), and (m, l) in
    // sml[u][lane]; the wave's own LDS reads of the region precede these
    // writes in order
    if (u <= last) {
        f32x4* w = reinterpret_cast<f32x4*>(region) + lane;
#pragma unroll
        for (int e = 0; e < 16; ++e)
            w[64 * e] = f32x4{o[e >> 2][4 * (e & 3)], o[e >> 2][4 * (e & 3) + 1],
                              o[e >> 2][4 * (e & 3) + 2], o[e >> 2][4 * (e & 3) + 3]};
        sml[u][lane] = f32x2{m_unit, l_unit};
    }
    __syncthreads();
    const int dt = wave >> 1;
    const int e0 = 4 * dt + 2 * (wave & 1);  // this wave's two state words
    float m = -INFINITY, l = 0.f;
    f32x4 acc[2] = {f32x4{}, f32x4{}};
    for (uint32_t w2 = 0; w2 <= last; ++w2) {
        const f32x4* w = reinterpret_cast<const f32x4*>(lds + w2 * kSkRegion) + lane;
        const f32x2 ml = sml[w2][lane];
        const f32x4 o0 = w[64 * e0], o1 = w[64 * (e0 + 1)];
        const float mx = fmaxf(m, ml[0]);  // ml[0] is finite
        const float a1 = fast_exp2(m - mx), a2 = fast_exp2(ml[0] - mx);
        l = l * a1 + ml[1] * a2;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            acc[0][e] = acc[0][e] * a1 + o0[e] * a2;
            acc[1][e] = acc[1][e] * a1 + o1[e] * a2;
        }
        m = mx;
    }
    const float inv = 1.f / add_xor<32>(l);
    if (query < N) {
        f16* orow = a.out + ((uint64_t)query * a.num_heads + head) * kD;
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int i4 = 2 * (wave & 1) + k;
            f16x4 w;
#pragma unroll
            for (int e = 0; e < 4; ++e) w[e] = (f16)(acc[k][e] * inv);
            *reinterpret_cast<f16x4*>(orow + 32 * dt + 8 * i4 + 4 * hh) = w;
        }
    }
}

// Split keys over 4 waves for prompts longer than the all-tiles-staged forms
// take.  A workgroup is ONE head's 32-query tile t (keys 0 .. 32 t + 31 in
// 32-key units 0 .. t); wave w owns units w, w + 4, w + 8, ... and streams
// them through two 16 KiB LDS buffers of its own (K and V swizzled as above):
// the copy of its unit k + 2 goes out once unit k is computed, and it waits
// for its own copies only (vmcnt), so the waves run without barriers until
// the combine.  Each wave keeps an online softmax with the lazy rescale of
// the long-prompt kernel; at the end the states meet in LDS as in the other
// split-keys forms (wave w folds output dims 32 w .. 32 w + 31).  Against
// the 4-head workgroups of prefill_d128<4, false, false>: four times the
// workgroups and a quarter of each one's chain, at four times the K/V reads
// (one head per workgroup instead of 4).
constexpr int kSknWaves = 4;
// automatic up to this many tokens: from 257 tokens (beyond the all-tiles
// forms) it measured 25-35 % faster than the 4-head workgroups (288 tokens
// 7.3 against 10.4 us, 1024 tokens 17.9 against 23.4 us), level at 1536
// (32.0 against 32.4 us) and slower from 1664 (37.0 against 34.6 us), where
// the 4x K/V reads of one-head workgroups outweigh their parallelism; from
// 1025 tokens the key-halves tile is faster (1152 tokens 23.6 against 26.8 us)
constexpr uint32_t kSknMaxTokens = 1024;
constexpr int kSknUnitBytes = 2 * kSkUnit * kD * 2;       // K + V of 32 keys: 16 KiB
constexpr int kSknDma = kSknUnitBytes / 1024;             // 16: 8 for K, then 8 for V

__global__ __launch_bounds__(64 * kSknWaves, 1) void prefill_skn(PrefillArgs a) {
    // per wave two unit buffers: [wave][2][16 KiB]
    __shared__ __attribute__((aligned(16))) char ub[kSknWaves * 2 * kSknUnitBytes];
    __shared__ f32x2 sml[kSknWaves][64];  // each wave's (m, l)
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n = lane & 31;
    const int hh = lane >> 5;
    uint32_t head, tile;
    if (!map_block(blockIdx.x, a.num_heads, a.q_tiles, head, tile)) return;
    const uint32_t last = tile;  // the diagonal unit
    if (last == 0 && wave != 0) return;  // one unit: wave 0 finishes it alone
    const uint32_t g = head / a.group;
    const uint32_t q0 = tile * (uint32_t)kSkUnit;
    const uint32_t N = a.seq_len;
    const uint32_t kv_row_bytes = (uint32_t)(a.kv_stride * 2);
    // units of this wave: wave, wave + 4, ... <= last
    const uint32_t nunits = (uint32_t)wave <= last ? (last - (uint32_t)wave) / kSknWaves + 1u : 0u;
    char* const mine = ub + wave * 2 * kSknUnitBytes;
    const uint32_t mine_lds = lds_addr(mine);

    f32x16 o[4];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) o[dt] = f32x16{};
    float m_used = -INFINITY, l_run = 0.f;

    // per-lane source offsets of the 16 copy instructions of a unit (K rows
    // 4 i + lane / 16 for i < 8, then V rows): the same for every unit
    uint32_t koff[kSknDma / 2], voff[kSknDma / 2];
#pragma unroll
    for (int i = 0; i < kSknDma / 2; ++i) {
        const uint32_t q = (uint32_t)i * 64u + (uint32_t)lane;
        const uint32_t r = q / kKChunks, c = q % kKChunks;
        koff[i] = r * kv_row_bytes + k_src_chunk(r, c) * 16u;
        voff[i] = r * kv_row_bytes + v_src_chunk(r, c) * 16u;
    }
    // copy unit u into buffer `buf` (K, then V); issued as inline assembly,
    // so the only waits for it are the explicit vmcnt waits below
    auto issue = [&](uint32_t u, uint32_t buf) {
        const uint32_t kv0 = u * (uint32_t)kSkUnit;  // < N: u <= last and q0 < N
        const uint32_t bytes = (N - kv0 - 1u) * kv_row_bytes + kD * 2;
        const u32x4 rk = rsrc_words(a.k + (uint64_t)kv0 * a.kv_stride + (uint64_t)g * kD, bytes);
        const u32x4 rv = rsrc_words(a.v + (uint64_t)kv0 * a.kv_stride + (uint64_t)g * kD, bytes);
        const uint32_t dst = __builtin_amdgcn_readfirstlane(mine_lds + buf * kSknUnitBytes);
#pragma unroll
        for (int i = 0; i < kSknDma / 2; ++i) dma16(rk, dst + 1024u * i, koff[i]);
#pragma unroll
        for (int i = 0; i < kSknDma / 2; ++i) dma16(rv, dst + 1024u * (kSknDma / 2 + i), voff[i]);
    };

    f16x8 qb[8];
    const uint32_t grp = (uint32_t)lane >> 4, jl = (uint32_t)lane & 15u;
    const uint32_t vrd = (4u * hh + (jl >> 2)) * kVP + 16u * (grp & 1u) + 4u * (jl & 3u);
    // unit k is in buffer k % 2; while it is computed, unit k + 1's copy (16
    // loads) may be in flight; once computed, its buffer takes unit k + 2.
    // Unit 0 is peeled off the loop: the compiler's own waits for the Q loads
    // (it does not see the copies, which its vmcnt values would then also
    // drain) stay out of the loop.
    auto step = [&](uint32_t k) {
        if (k + 1 < nunits) __builtin_amdgcn_s_waitcnt(vmcnt_imm(kSknDma));
        else __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
        const uint32_t u = (uint32_t)wave + kSknWaves * k;
        const f16* kt = reinterpret_cast<const f16*>(mine + (k & 1u) * kSknUnitBytes);
        const f16* vt = kt + kSkUnit * kD;
        // S^T = K . Q^T, online softmax, O^T += V^T . P^T
        f32x16 s = f32x16{};
#pragma unroll
        for (int ks = 0; ks < 8; ++ks)
            s = mfma32(lds16(kt + k_read_offset((uint32_t)n, (uint32_t)hh, (uint32_t)ks)), qb[ks], s);
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            float x = s[i];
            if (u == last) {
                // the diagonal unit starts at q0: mask keys past the query and past N
                const uint32_t key = q0 + 8u * (uint32_t)(i >> 2) + 4u * hh + (uint32_t)(i & 3);
                if (key > q0 + n || key >= N) x = -INFINITY;
                s[i] = x;
            }
            mx = fmaxf(mx, x);
        }
        // the pair's exchange only in the rescale block, as in prefill_d128
        const float m_lane = mx * a.scale_log2;
        if (__any(m_lane > m_used + kRescaleSlack)) {
            const float m_tile = max_xor<32>(m_lane);
            const float mn = (m_tile > m_used + kRescaleSlack) ? m_tile : m_used;
            const float al = fast_exp2(m_used - mn);
            l_run *= al;
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) o[dt] *= al;
            m_used = mn;
        }
        const float mneg = -m_used;
        float psum = 0.f;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            f16x8 va[4];
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) {
                const uint32_t vd = vrd + 32u * ((uint32_t)dt ^ (jl >> 2));
                const f16x4 lo = lds_tr4(vt + vd + 16 * ks * kVP);
                const f16x4 hi = lds_tr4(vt + vd + (16 * ks + 8) * kVP);
                va[dt] = f16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            }
            f16x8 pb;
#pragma unroll
            for (int r = 0; r < 8; ++r)
                pb[r] = (f16)fast_exp2(__builtin_fmaf(s[8 * ks + r], a.scale_log2, mneg));
#pragma unroll
            for (int r = 0; r < 8; r += 2) {
                const f16x2 pair = {pb[r], pb[r + 1]};
                psum = __builtin_amdgcn_fdot2(pair, f16x2{(f16)1.0f, (f16)1.0f}, psum, false);
            }
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) o[dt] = mfma32(va[dt], pb, o[dt]);
        }
        l_run += psum;
        // the unit's LDS reads have returned (their MFMAs consumed them), so
        // its buffer can take unit k + 2
        if (k + 2 < nunits) issue(u + 2u * kSknWaves, k & 1u);
    };
    // everything that uses Q in one block: the compiler's waits for the Q
    // loads then stay in the peeled first unit on every path into the loop
    if (nunits) {
        // Q^T B operands (lane (hh, n): Q[q0 + n][head][16 s + 8 hh .. +7]),
        // issued before the first copies; rows past N read as zero
        const uint32_t q_row_bytes = (uint32_t)(a.q_stride * 2);
        const BufRsrc rq = make_rsrc(a.q + (uint64_t)head * kD,
                                     __builtin_amdgcn_readfirstlane((N - 1) * q_row_bytes + kD * 2));
        const uint32_t qoff = (q0 + n) * q_row_bytes + 16u * hh;
#pragma unroll
        for (int s = 0; s < 8; ++s) qb[s] = buf_ld16(rq, qoff + 32u * s);
        issue((uint32_t)wave, 0u);
        if (nunits > 1) issue((uint32_t)wave + kSknWaves, 1u);
        step(0);
        for (uint32_t k = 1; k < nunits; ++k) step(k);
    }

    const uint32_t query = q0 + n;
    if (last == 0) {
        const float inv = 1.f / add_xor<32>(l_run);
        if (query < N) {
            f16* orow = a.out + ((uint64_t)query * a.num_heads + head) * kD;
#pragma unroll
            for (int dt = 0; dt < 4; ++dt)
#pragma unroll
                for (int i4 = 0; i4 < 4; ++i4) {
                    f16x4 w;
#pragma unroll
                    for (int e = 0; e < 4; ++e) w[e] = (f16)(o[dt][4 * i4 + e] * inv);
                    *reinterpret_cast<f16x4*>(orow + 32 * dt + 8 * i4 + 4 * hh) = w;
                }
        }
        return;
    }
    // The waves with units (0 .. min(3, last)) leave O^T in their buffer 0
    // (16 KiB = 16 words x 64 lanes; every copy has landed and every read of
    // it is done) and (m, l) in sml; m is finite (each wave's first unit
    // holds a key <= every query of the tile).  Wave w then folds dims
    // 32 w .. 32 w + 31 of every state.
    const uint32_t nstates = last < (uint32_t)kSknWaves ? last + 1u : (uint32_t)kSknWaves;
    if (nunits) {
        f32x4* w = reinterpret_cast<f32x4*>(mine) + lane;
#pragma unroll
        for (int e = 0; e < 16; ++e)
            w[64 * e] = f32x4{o[e >> 2][4 * (e & 3)], o[e >> 2][4 * (e & 3) + 1],
                              o[e >> 2][4 * (e & 3) + 2], o[e >> 2][4 * (e & 3) + 3]};
        sml[wave][lane] = f32x2{m_used, l_run};
    }
    __syncthreads();
    const int dt = wave;
    float m = -INFINITY, l = 0.f;
    f32x16 acc = f32x16{};
    for (uint32_t w2 = 0; w2 < nstates; ++w2) {
        const f32x4* w = reinterpret_cast<const f32x4*>(ub + w2 * 2 * kSknUnitBytes) + lane;
        const f32x2 ml = sml[w2][lane];
        f32x4 ow[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) ow[q] = w[64 * (4 * dt + q)];
        const float mx = fmaxf(m, ml[0]);  // ml[0] is finite
        const float a1 = fast_exp2(m - mx), a2 = fast_exp2(ml[0] - mx);
        l = l * a1 + ml[1] * a2;
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[i] = acc[i] * a1 + ow[i >> 2][i & 3] * a2;
        m = mx;
    }
    const float inv = 1.f / add_xor<32>(l);
    if (query < N) {
        f16* orow = a.out + ((uint64_t)query * a.num_heads + head) * kD;
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4) {
            f16x4 w;
#pragma unroll
            for (int e = 0; e < 4; ++e) w[e] = (f16)(acc[4 * i4 + e] * inv);
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

// 4-wave workgroups up to this many tokens (see prefill_d128): with the MFMA
// results in VGPRs, measured 8-20 % faster than 8-wave ones from 1664 to
// 5120 tokens and 2-5 % at 6144 (162 against 170 us); from 7168 tokens the
// 8-wave tile wins (205 against 222 us; 258 against 285 us at 8192), its two
// waves per SIMD hiding each other's softmax once every CU has work
constexpr uint32_t kFourWaveMaxTokens = 6144;

// 32-query tiles whose key tiles two 4-wave groups split
// (prefill_d128<8, false, false, true>), automatic in (kKhMinTokens,
// kKhMaxTokens]: a 32-query workgroup's chain of steps is half its chain of
// key tiles, so the long chains near the end of a mid-length prompt no
// longer leave CUs idle once the short ones are done.  Measured against the
// default forms on one box: 1152 tokens 23.6 against 26.8 us (prefill_skn),
// 1536 27.6 against 33.3, 2048 35.0 against 39.4, 3072 53.0 against 63.9,
// 4096 81.6 against 91.7 (4-wave tiles); 1024 tokens 21.8 against 20.0
// (prefill_skn), 4608 110.5 against 108.3, 6144 177.4 against 166.7, 8192
// 288 against 266 us (the 8-wave tile shares each K/V tile between twice the
// queries).
constexpr uint32_t kKhMinTokens = 1024;
constexpr uint32_t kKhMaxTokens = 4096;

hipError_t launch_prefill_kernel(const PrefillArgs& a0, int path, hipStream_t stream) {
    if (path != 1) return hipErrorInvalidValue;
    const long wopt = get_option(kOptPrefillWaves);
    const int waves = wopt == 4 || wopt == 8 ? (int)wopt
                                              : (a0.seq_len <= kFourWaveMaxTokens ? 4 : 8);
    PrefillArgs a = a0;
    const uint32_t bm = 8u * (uint32_t)waves;  // query tokens per workgroup
    a.q_tiles = (a.seq_len + bm - 1) / bm;
    const uint32_t quads = a.num_heads / 4u;
    uint64_t blocks;
    if (quads <= 8 && (8 % quads) == 0) {
        const uint32_t per = 8u / quads;
        blocks = 8ull * ((a.q_tiles + per - 1) / per);
    } else {
        blocks = (uint64_t)a.q_tiles * quads;
    }
    if (blocks > 0x7fffffffull) return hipErrorInvalidValue;
    const bool all = waves == 4 && a.seq_len <= kAllTiles * kBN &&
                     get_option(kOptPrefillStageAll) != 1;
    const long sk_opt = get_option(kOptPrefillSplitKeys);
    const long kh_opt = get_option(kOptPrefillKeyHalves);
    const bool kh = kh_opt == 2 || (kh_opt == 0 && sk_opt == 0 && wopt == 0 &&
                                    a0.seq_len > kKhMinTokens && a0.seq_len <= kKhMaxTokens);
    if (kh) {
        // 32-query tiles x 4 heads, 8 waves: the two 4-wave groups split the
        // key tiles
        PrefillArgs b = a0;
        b.q_tiles = (b.seq_len + 31u) / 32u;
        uint64_t kh_blocks;
        if (quads <= 8 && (8 % quads) == 0) {
            const uint32_t per = 8u / quads;
            kh_blocks = 8ull * ((b.q_tiles + per - 1) / per);
        } else {
            kh_blocks = (uint64_t)b.q_tiles * quads;
        }
        if (kh_blocks > 0x7fffffffull) return hipErrorInvalidValue;
        hipLaunchKernelGGL((prefill_d128<8, false, false, true>), dim3((uint32_t)kh_blocks),
                           dim3(512), 0, stream, b);
        return hipGetLastError();
    }
    const bool skn = sk_opt == 4 || (sk_opt == 0 && wopt == 0 && a0.seq_len > kAllTiles * kBN &&
                                     a0.seq_len <= kSknMaxTokens);
    if (skn) {
        // one 4-wave workgroup per (head, 32-query tile), 32-key units streamed per wave
        PrefillArgs b = a0;
        b.q_tiles = (b.seq_len + kSkUnit - 1) / kSkUnit;
        const uint64_t n_blocks = (uint64_t)b.q_tiles * b.num_heads;
        if (n_blocks > 0x7fffffffull) return hipErrorInvalidValue;
        hipLaunchKernelGGL(prefill_skn, dim3((uint32_t)n_blocks), dim3(64 * kSknWaves), 0, stream,
                           b);
        return hipGetLastError();
    }
    const bool sk = all && sk_opt != 1;
    // 32-key units over 8 waves only where one query tile needs no combine
    // (N <= 32: 4.1 against 4.6 us per graph launch); with several units
    // their 8 fp32 states cost twice the LDS traffic of the 4-wave form's
    // (N = 254: 7.1 against 6.6 us)
    const bool sk32 = sk && (sk_opt == 3 || (sk_opt != 2 && a.seq_len <= kSkUnit)) &&
                      a.seq_len <= kSkMaxTokens;
    if (sk32) {
        // one 8-wave workgroup per (head, 32-query tile), 32 keys per wave
        PrefillArgs b = a0;
        b.q_tiles = (b.seq_len + kSkUnit - 1) / kSkUnit;
        hipLaunchKernelGGL(prefill_sk32, dim3(b.q_tiles * b.num_heads), dim3(64 * kSkWaves), 0,
                           stream, b);
    } else if (sk) {
        // one workgroup per (head, 32-query tile)
        const uint64_t sk_blocks = (uint64_t)a.q_tiles * a.num_heads;
        if (sk_blocks > 0x7fffffffull) return hipErrorInvalidValue;
        hipLaunchKernelGGL((prefill_d128<4, true, true>), dim3((uint32_t)sk_blocks), dim3(256), 0,
                           stream, a);
    } else if (all)
        hipLaunchKernelGGL((prefill_d128<4, true, false>), dim3((uint32_t)blocks), dim3(256), 0,
                           stream, a);
    else if (waves == 4)
        hipLaunchKernelGGL((prefill_d128<4, false, false>), dim3((uint32_t)blocks), dim3(256), 0,
                           stream, a);
    else
        hipLaunchKernelGGL((prefill_d128<8, false, false>), dim3((uint32_t)blocks), dim3(512), 0,
                           stream, a);
    return hipGetLastError();
}

}  // namespace attn
