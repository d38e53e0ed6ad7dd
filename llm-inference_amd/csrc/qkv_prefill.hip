// Prefill QKV projection for gfx950 on fp16 MFMA, optionally with the RoPE +
// KV-cache append of the same tokens folded into its epilogue.
//
// Reference semantics: launch_qkv_gemm (qkv_gemm.hip.cpp:7-105) is the
// rocBLAS product Y[M][N] = X[M][K] . W[N][K]^T (fp16 in, fp32 compute, fp16
// out; X = the normalised hidden states of M tokens, W = the Q rows of all
// heads, then K, then V).  The engine then runs launch_rope_and_store_kv on Y
// (model_inference.hpp:266-285): Q heads rotated in place, K rotated into
// cache rows start_pos + t (Y's K left unrotated), V copied; NoPE layers copy
// K and V only.
//
// MFMA path (K a multiple of 64, X and W 16-byte aligned):
//  * workgroup = a BM x 128 tile of Y (BM = 64 * WMT tokens, 128 output
//    features = one head when D = 128), 4 waves as 2 (tokens) x 2 (features),
//    each wave 32*WMT tokens x 64 features on v_mfma_f32_32x32x16_f16.  A
//    wave's 64 features are columns c and c + 64 of the head (c = 32 * wave
//    column + lane % 32), so both halves of every rotation pair sit in the same
//    lane and the fused epilogue rotates in registers.
//  * X and W tiles of 64 k-values are copied straight from global memory into
//    LDS by buffer_load ... lds (no VGPRs, no LDS stores), three stages deep,
//    one barrier per stage.  LDS rows are 128 B with the 16-byte chunks of row
//    r stored at position chunk ^ ((r >> 1) & 7), so the MFMA operand reads
//    (16 rows x 16 B per pass) hit 16 distinct bank groups; the DMA source of
//    each lane is chosen to produce that order.  Rows past M or N read as zero
//    through the buffer range check.
//  * Workgroups are dispatched round-robin over the 8 XCDs; the tile grid is
//    split over them (2 x 4 when it divides: each XCD owns half the token
//    tiles and a quarter of the feature tiles, whose W rows stay in its L2).
//  * From 7168 tokens (N a multiple of 384, Y 16-byte aligned) a 256 x 384
//    tile of 8 waves (qkv_gemm_wide, below) replaces it: a third of the X
//    re-reads and 1.5x the MFMA work per staged byte; identical results.
//  * Epilogue: fp32 -> fp16 (the GEMM's output rounding), then for the fused
//    kernel the rope.hip.cpp:44-58 rotation on those fp16 values (fp32
//    products each rounded, no contraction): Q rows written rotated, K rows
//    unrotated plus rotated into the cache, V rows plus their cache copy --
//    the bytes of the two-launch sequence on the same GEMM output.
#include "attn_internal.hpp"

namespace attn {

namespace {

constexpr int kBK = 64;      // k-values per stage
// automatic use of the wide tile: from 28 token tiles (224 of the 256 CUs
// busy at N = 3072); below that the 256 x 128 tile keeps more CUs busy
constexpr uint32_t kWideMinTokens = 7168;
constexpr int kRowH = kBK;   // halves per LDS row (128 B, no padding)
constexpr int kThreads = 256;

#define LDS_AS __attribute__((address_space(3)))

__device__ __forceinline__ f16x8 lds16(const f16* p) {
    return *reinterpret_cast<const f16x8*>(p);
}

__device__ __forceinline__ f32x16 mfma32(f16x8 a, f16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// blockIdx -> (token tile, feature tile).  Workgroups are dispatched
// round-robin over the 8 XCDs (bid % 8), each with its own L2.  When the tile
// grid splits 2 x 4, XCD x owns token half x / 4 and feature quarter x % 4
// (SmolLM3 at 8192 tokens: 16 token tiles x 6 feature tiles, 16 MB of X and
// 3 MB of W per XCD, so W stays in L2 and each X tile is fetched once per
// XCD); otherwise, when the feature tiles divide by 8, XCD x owns feature
// tiles x, x + 8, ... and walks all token tiles.
__device__ __forceinline__ void map_tile(uint32_t bid, uint32_t m_tiles, uint32_t n_tiles,
                                         uint32_t& mt, uint32_t& nt) {
    if ((m_tiles & 1u) == 0 && (n_tiles & 3u) == 0) {
        const uint32_t xcd = bid & 7u, j = bid >> 3;
        const uint32_t nm = m_tiles >> 1, nn = n_tiles >> 2;
        const uint32_t ml = j / nn;
        mt = (xcd >> 2) * nm + ml;
        nt = (xcd & 3u) * nn + (j - ml * nn);
    } else if ((n_tiles & 7u) == 0) {
        const uint32_t per = n_tiles >> 3;
        const uint32_t xcd = bid & 7u, j = bid >> 3;
        mt = j / per;
        nt = xcd + 8u * (j - mt * per);
    } else {
        mt = bid / n_tiles;
        nt = bid - mt * n_tiles;
    }
}

template <int WMT, bool FUSED>
__global__ __launch_bounds__(kThreads, 1) void qkv_gemm_mfma(QkvGemmArgs a) {
    constexpr int BM = 64 * WMT;
    constexpr int kADma = BM * 8 / 64;        // 1 KiB DMA instructions per X stage
    constexpr int kBDma = 128 * 8 / 64;       // ... per W stage (16)
    constexpr int kDmaPerWave = (kADma + kBDma) / 4;
    // vmcnt value that leaves one stage of this wave's DMA outstanding
    constexpr int kWaitOne = 0x0F70 | (kDmaPerWave & 15) | ((kDmaPerWave >> 4) << 14);
    static_assert(kDmaPerWave < 64, "vmcnt range");

    // three stages; the DMA is issued by dma16 (inline assembly), so the only
    // waits between stages are the explicit vmcnt + barrier of each step
    __shared__ __attribute__((aligned(16))) f16 sa0[BM * kRowH];
    __shared__ __attribute__((aligned(16))) f16 sa1[BM * kRowH];
    __shared__ __attribute__((aligned(16))) f16 sa2[BM * kRowH];
    __shared__ __attribute__((aligned(16))) f16 sb0[128 * kRowH];
    __shared__ __attribute__((aligned(16))) f16 sb1[128 * kRowH];
    __shared__ __attribute__((aligned(16))) f16 sb2[128 * kRowH];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const uint32_t n = (uint32_t)lane & 31u, hh = (uint32_t)lane >> 5;

    uint32_t m_tile, n_tile;
    map_tile(blockIdx.x, a.m_tiles, a.n_tiles, m_tile, n_tile);
    // uniform by construction; keeps the buffer resources in SGPRs
    m_tile = __builtin_amdgcn_readfirstlane(m_tile);
    n_tile = __builtin_amdgcn_readfirstlane(n_tile);
    const uint32_t m0 = m_tile * BM, n0 = n_tile * 128u;
    const uint32_t K = a.K;
    const uint32_t row_bytes = K * 2u;
    const uint32_t rows_x = a.M - m0;                       // >= 1
    const uint32_t rows_w = a.N > n0 ? a.N - n0 : 0u;       // >= 1 by the grid
    const f16* xb = a.x + (uint64_t)m0 * K;
    const f16* wb = a.w + (uint64_t)n0 * K;

    // A wave's DMA instructions t < kADma / 4 fill X-buffer bytes [1024 i,
    // 1024 i + 1024) with i = wave + 4 t, the others W-buffer bytes with
    // i = wave + 4 (t - kADma / 4); lane L writes 16-byte position p = 64 i + L:
    // row p / 8, slot p % 8, which holds chunk slot ^ ((row >> 1) & 7).
    constexpr int kATs = kADma / 4;
    static_assert(kADma % 4 == 0, "X DMA instructions split evenly over 4 waves");
    uint32_t voff[kDmaPerWave];
#pragma unroll
    for (int t = 0; t < kDmaPerWave; ++t) {
        const uint32_t ip = (uint32_t)(wave + 4 * (t < kATs ? t : t - kATs));
        const uint32_t p = 64u * ip + (uint32_t)lane;
        const uint32_t row = p >> 3, slot = p & 7u;
        voff[t] = row * row_bytes + 16u * (slot ^ ((row >> 1) & 7u));
    }
    auto stage = [&](uint32_t kt, f16* sa, f16* sb) {
        // resources start at k-value 64 kt of the tile's first row and end at
        // the last row of the matrix: rows past M / N read as zero
        const uint32_t k0b = kt * (uint32_t)kBK * 2u;
        const u32x4 rx = rsrc_words(reinterpret_cast<const char*>(xb) + k0b,
                                    rows_x * row_bytes - k0b);
        const u32x4 rw = rsrc_words(reinterpret_cast<const char*>(wb) + k0b,
                                    rows_w * row_bytes - k0b);
        const uint32_t la = lds_addr(sa) + 1024u * (uint32_t)wave;
        const uint32_t lb = lds_addr(sb) + 1024u * (uint32_t)wave;
#pragma unroll
        for (int t = 0; t < kDmaPerWave; ++t) {
            if (t < kATs)
                dma16(rx, la + 4096u * t, voff[t]);
            else
                dma16(rw, lb + 4096u * (t - kATs), voff[t]);
        }
    };

    f32x16 acc[WMT][2];
#pragma unroll
    for (int mt = 0; mt < WMT; ++mt) acc[mt][0] = acc[mt][1] = f32x16{};

    // operand rows of this lane: X rows wm*32*WMT + 32 mt + n, W rows
    // 64 nt + 32 wn + n; all start at a multiple of 32 plus n, so the chunk
    // swizzle (row >> 1) & 7 is (n >> 1) & 7 for every operand
    const uint32_t sw = (n >> 1) & 7u;
    const uint32_t a_row0 = (uint32_t)wm * 32u * WMT + n;
    const uint32_t b_row0 = 32u * (uint32_t)wn + n;

    auto compute = [&](const f16* sa, const f16* sb) {
        f16x8 af[2][WMT], bf[2][2];
        auto fetch = [&](int ks, int buf) {
            const uint32_t pos = 8u * (((uint32_t)(2 * ks) + hh) ^ sw);
#pragma unroll
            for (int mt = 0; mt < WMT; ++mt)
                af[buf][mt] = lds16(sa + (a_row0 + 32u * mt) * kRowH + pos);
#pragma unroll
            for (int nt = 0; nt < 2; ++nt)
                bf[buf][nt] = lds16(sb + (b_row0 + 64u * nt) * kRowH + pos);
        };
        fetch(0, 0);
#pragma unroll
        for (int ks = 0; ks < kBK / 16; ++ks) {
            const int cur = ks & 1;
            if (ks + 1 < kBK / 16) fetch(ks + 1, cur ^ 1);
#pragma unroll
            for (int mt = 0; mt < WMT; ++mt)
#pragma unroll
                for (int nt = 0; nt < 2; ++nt)
                    acc[mt][nt] = mfma32(af[cur][mt], bf[cur][nt], acc[mt][nt]);
        }
        // schedule: the operand reads of k-step ks + 1 interleaved with the
        // MFMAs of k-step ks, so one wave per SIMD keeps the MFMA pipe fed
        // while its LDS reads are in flight
        constexpr int kReads = WMT + 2, kMfmas = 2 * WMT;
        __builtin_amdgcn_sched_group_barrier(0x100, kReads, 0);
#pragma unroll
        for (int ks = 0; ks + 1 < kBK / 16; ++ks) {
#pragma unroll
            for (int i = 0; i < (kReads > kMfmas ? kReads : kMfmas); ++i) {
                if (i < kMfmas) __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                if (i < kReads) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            }
        }
        __builtin_amdgcn_sched_group_barrier(0x008, kMfmas, 0);
    };

    // stage kt sits in buffer kt % 3; at the top of step kt this wave has
    // stages kt and kt + 1 in flight: wait for kt, then the barrier makes
    // every wave's copy of it visible and frees buffer (kt + 2) % 3 (last
    // read in step kt - 1) for the DMA of stage kt + 2
    const uint32_t KT = K / kBK;
    if (KT > 0) stage(0, sa0, sb0);
    if (KT > 1) stage(1, sa1, sb1);
    // (a bare s_barrier: __syncthreads' fence would also wait for stage kt + 1)
    auto step = [&](uint32_t kt, const f16* sa, const f16* sb, f16* na, f16* nb) {
        asm volatile("" ::: "memory");
        if (kt + 1 < KT)
            __builtin_amdgcn_s_waitcnt(kWaitOne);
        else
            __builtin_amdgcn_s_waitcnt(0x0F70);
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        if (kt + 2 < KT) stage(kt + 2, na, nb);
        compute(sa, sb);
    };
    for (uint32_t kt = 0; kt < KT; kt += 3) {
        step(kt, sa0, sb0, sa2, sb2);
        if (kt + 1 < KT) step(kt + 1, sa1, sb1, sa0, sb0);
        if (kt + 2 < KT) step(kt + 2, sa2, sb2, sa1, sb1);
    }

    // ---- epilogue.  acc[mt][nt][r] is token m0 + wm*32*WMT + 32 mt + 8 (r / 4)
    // + 4 hh + r % 4, feature n0 + 64 nt + c with c = 32 wn + n.  The fp16
    // tile goes through LDS (features 0..63 in sa0, 64..127 in sa1, both
    // [BM][64]) so that every global store is 16 bytes: 8 threads per token
    // row, thread j holding features 8j..8j+7 and 64+8j..64+8j+7 -- the two
    // halves of 8 rotation pairs.
    const uint32_t c = 32u * (uint32_t)wn + n;
    __syncthreads();  // every wave is done with the stage buffers
#pragma unroll
    for (int mt = 0; mt < WMT; ++mt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const uint32_t row = a_row0 - n + 32u * mt + 8u * (r >> 2) + 4u * hh + (r & 3);
            sa0[row * 64u + c] = (f16)acc[mt][0][r];
            sa1[row * 64u + c] = (f16)acc[mt][1][r];
        }
    __syncthreads();
    const uint32_t N = a.N;
    const uint32_t j8 = 8u * ((uint32_t)tid & 7u), rsub = (uint32_t)tid >> 3;
    if (!FUSED) {
#pragma unroll
        for (int p = 0; p < BM / 32; ++p) {
            const uint32_t row = 32u * p + rsub, m = m0 + row;
            if (m >= a.M) break;
            const f16x8 lo = lds16(sa0 + row * 64u + j8);
            const f16x8 hi = lds16(sa1 + row * 64u + j8);
            f16* yr = a.y + (uint64_t)m * N + n0;
            if (a.vec_out) {  // N % 8 == 0: a chunk is wholly inside or outside
                if (n0 + j8 < N) st16(yr + j8, lo);
                if (n0 + 64u + j8 < N) st16(yr + 64u + j8, hi);
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    if (n0 + j8 + e < N) yr[j8 + e] = lo[e];
                    if (n0 + 64u + j8 + e < N) yr[64u + j8 + e] = hi[e];
                }
            }
        }
        return;
    }
    // fused: the tile is head n_tile (D = 128, N = (Hq + 2 Hkv) * 128)
    const uint32_t head = n_tile;
    const uint32_t Hq = a.num_heads, Hkv = a.num_kv_heads;
    const uint64_t kv_dim = (uint64_t)Hkv * 128u;
    const bool is_q = head < Hq;
    const bool is_k = !is_q && head < Hq + Hkv;
    const bool rot = a.apply != 0 && (is_q || is_k);
    f16* cache = is_q ? nullptr
                      : (is_k ? a.kc + (uint64_t)(head - Hq) * 128u
                              : a.vc + (uint64_t)(head - Hq - Hkv) * 128u);
    // table rows of all passes first (rows past M read row M - 1, unused)
    f16x8 cs[BM / 32], sn[BM / 32];
    if (rot) {
#pragma unroll
        for (int p = 0; p < BM / 32; ++p) {
            const uint32_t m = min(m0 + 32u * p + rsub, a.M - 1u);
            const uint64_t t = ((uint64_t)a.start_pos + m) * 64u + j8;
            cs[p] = ld16(a.cos_t + t);
            sn[p] = ld16(a.sin_t + t);
        }
    }
#pragma unroll
    for (int p = 0; p < BM / 32; ++p) {
        const uint32_t row = 32u * p + rsub, m = m0 + row;
        if (m >= a.M) break;
        const f16x8 lo = lds16(sa0 + row * 64u + j8);
        const f16x8 hi = lds16(sa1 + row * 64u + j8);
        f16x8 r0 = lo, r1 = hi;
        if (rot) rope_rotate8(lo, hi, cs[p], sn[p], r0, r1);
        f16* yr = a.y + (uint64_t)m * N + n0;
        const uint64_t pos = (uint64_t)a.start_pos + m;
        if (is_q) {
            st16(yr + j8, r0);
            st16(yr + 64u + j8, r1);
        } else {
            st16(yr + j8, lo);
            st16(yr + 64u + j8, hi);
            f16* cr = cache + pos * kv_dim;
            st16(cr + j8, r0);
            st16(cr + 64u + j8, r1);
        }
    }
}

// Wide tile for long prompts: a workgroup computes 256 tokens x 384 features
// (three heads when D = 128) with 8 waves as 2 (tokens) x 4 (features), each
// wave 128 x 96 on v_mfma_f32_32x32x16_f16, so every X and W byte staged in
// LDS feeds 1.5x (X) and 3x (W) the MFMA work of the 256 x 128 tile and the
// X re-reads from L2 drop by two thirds.  64 k-values per stage (128-byte
// LDS rows, chunk c of row r at position c ^ ((r >> 1) & 7): conflict-free
// operand reads), two stages of 80 KiB (all of the LDS; the DMA of stage
// kt + 1 runs under the MFMAs of stage kt; 6 % faster than three stages of
// 32 k-values, which need twice the barriers).  Each output sums its 16-value
// k-chunks in the same order as qkv_gemm_mfma, so the two kernels give
// identical bits.
// The epilogue runs one head at a time through LDS with the qkv_gemm_mfma
// store pattern.
constexpr int kWBM = 256;
constexpr int kWBN = 384;
constexpr int kWBK = 64;
constexpr int kWThreads = 512;
constexpr int kWADma = kWBM * 8 / 64;                  // 1 KiB DMA instructions per X stage (32)
constexpr int kWBDma = kWBN * 8 / 64;                  // ... per W stage (48)
constexpr int kWATs = kWADma / 8;                      // X instructions per wave (4)
constexpr int kWDmaPerWave = (kWADma + kWBDma) / 8;    // 10
constexpr uint32_t kWStageA = kWBM * kWBK * 2;         // bytes of X per stage
constexpr uint32_t kWStage = kWStageA + kWBN * kWBK * 2;  // bytes per stage (80 KiB)

template <bool FUSED>
__global__ __launch_bounds__(kWThreads, 1) void qkv_gemm_wide(QkvGemmArgs a) {
    __shared__ __attribute__((aligned(16))) f16 lds[2 * kWStage / 2];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 2, wn = wave & 3;
    const uint32_t n = (uint32_t)lane & 31u, hh = (uint32_t)lane >> 5;

    uint32_t m_tile, n_tile;
    map_tile(blockIdx.x, a.m_tiles, a.n_tiles, m_tile, n_tile);
    m_tile = __builtin_amdgcn_readfirstlane(m_tile);
    n_tile = __builtin_amdgcn_readfirstlane(n_tile);
    const uint32_t m0 = m_tile * kWBM, n0 = n_tile * kWBN;
    const uint32_t K = a.K;
    const uint32_t row_bytes = K * 2u;
    const uint32_t rows_x = a.M - m0;   // >= 1
    const uint32_t rows_w = a.N - n0;   // = 384 (N is a multiple of 384)
    const f16* xb = a.x + (uint64_t)m0 * K;
    const f16* wb = a.w + (uint64_t)n0 * K;

    // DMA instruction t < 4 of a wave fills X bytes [1024 i, 1024 i + 1024)
    // with i = wave + 8 t, the others W bytes with i = wave + 8 (t - 4); lane L
    // writes 16-byte position p = 64 i + L: row p / 8, slot p % 8, which holds
    // chunk slot ^ ((row >> 1) & 7)
    uint32_t voff[kWDmaPerWave];
#pragma unroll
    for (int t = 0; t < kWDmaPerWave; ++t) {
        const uint32_t ip = (uint32_t)(wave + 8 * (t < kWATs ? t : t - kWATs));
        const uint32_t p = 64u * ip + (uint32_t)lane;
        const uint32_t row = p >> 3, slot = p & 7u;
        voff[t] = row * row_bytes + 16u * (slot ^ ((row >> 1) & 7u));
    }
    const uint32_t lds0 = lds_addr(lds);
    auto stage = [&](uint32_t kt) {
        const uint32_t k0b = kt * (uint32_t)kWBK * 2u;
        const u32x4 rx = rsrc_words(reinterpret_cast<const char*>(xb) + k0b,
                                    rows_x * row_bytes - k0b);
        const u32x4 rw = rsrc_words(reinterpret_cast<const char*>(wb) + k0b,
                                    rows_w * row_bytes - k0b);
        const uint32_t base = lds0 + (kt & 1u) * kWStage + 1024u * (uint32_t)wave;
#pragma unroll
        for (int t = 0; t < kWDmaPerWave; ++t) {
            if (t < kWATs)
                dma16(rx, base + 8192u * t, voff[t]);
            else
                dma16(rw, base + kWStageA + 8192u * (t - kWATs), voff[t]);
        }
    };

    f32x16 acc[4][3];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int nt = 0; nt < 3; ++nt) acc[mt][nt] = f32x16{};

    // operand rows: X rows 128 wm + 32 mt + n, W rows 96 wn + 32 nt + n; both
    // start at a multiple of 32 plus n, so the swizzle is (n >> 1) & 7
    const uint32_t sw = (n >> 1) & 7u;
    const uint32_t a_row0 = 128u * (uint32_t)wm + n;
    const uint32_t b_row0 = 96u * (uint32_t)wn + n;

    auto compute = [&](uint32_t kt) {
        const f16* sa = lds + (kt & 1u) * (kWStage / 2u);
        const f16* sb = sa + kWStageA / 2u;
#pragma unroll
        for (int ks = 0; ks < kWBK / 16; ++ks) {
            const uint32_t pos = 8u * (((uint32_t)(2 * ks) + hh) ^ sw);
            f16x8 af[4], bf[3];
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) af[mt] = lds16(sa + (a_row0 + 32u * mt) * kWBK + pos);
#pragma unroll
            for (int nt = 0; nt < 3; ++nt) bf[nt] = lds16(sb + (b_row0 + 32u * nt) * kWBK + pos);
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                for (int nt = 0; nt < 3; ++nt) acc[mt][nt] = mfma32(af[mt], bf[nt], acc[mt][nt]);
        }
    };

    // stage kt sits in buffer kt & 1: wait for this wave's copy of it, the
    // barrier makes every wave's copy visible and frees the other buffer
    // (read in step kt - 1) for the DMA of stage kt + 1
    const uint32_t KT = K / kWBK;
    if (KT > 0) stage(0);
    for (uint32_t kt = 0; kt < KT; ++kt) {
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        if (kt + 1 < KT) stage(kt + 1);
        compute(kt);
    }

    // ---- epilogue, one head (128 features) per round.  acc[mt][nt][r] is
    // token m0 + 128 wm + 32 mt + 8 (r / 4) + 4 hh + r % 4, tile feature
    // f = 96 wn + 32 nt + n; a 32-feature block never straddles two heads.
    f16* lo = lds;             // [256][64]: features 0..63 of the round's head
    f16* hi = lds + kWBM * 64; // [256][64]: features 64..127
    const uint32_t N = a.N;
    const uint32_t j8 = 8u * ((uint32_t)tid & 7u), rsub = (uint32_t)tid >> 3;
    const uint32_t Hq = a.num_heads, Hkv = a.num_kv_heads;
    const uint64_t kv_dim = (uint64_t)Hkv * 128u;
#pragma unroll 1
    for (uint32_t h = 0; h < 3; ++h) {
        __syncthreads();  // the stages (h = 0) or the previous round's tile are free
#pragma unroll
        for (int nt = 0; nt < 3; ++nt) {
            const uint32_t fb = 96u * (uint32_t)wn + 32u * (uint32_t)nt;  // block's first feature
            if (fb / 128u != h) continue;
            const uint32_t c = (fb & 127u) + n;
            f16* dst = (c < 64u ? lo : hi) + (c & 63u);
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const uint32_t row = 128u * (uint32_t)wm + 32u * mt + 8u * (r >> 2) + 4u * hh +
                                         (r & 3);
                    dst[row * 64u] = (f16)acc[mt][nt][r];
                }
        }
        __syncthreads();
        const uint32_t hn0 = n0 + 128u * h;  // first feature of the round's head
        if (!FUSED) {
#pragma unroll
            for (int p = 0; p < kWBM / 64; ++p) {
                const uint32_t row = 64u * p + rsub, m = m0 + row;
                if (m >= a.M) break;
                f16* yr = a.y + (uint64_t)m * N + hn0;
                st16(yr + j8, lds16(lo + row * 64u + j8));
                st16(yr + 64u + j8, lds16(hi + row * 64u + j8));
            }
            continue;
        }
        // fused: the round's tile is head hn0 / 128 (D = 128)
        const uint32_t head = hn0 / 128u;
        const bool is_q = head < Hq;
        const bool is_k = !is_q && head < Hq + Hkv;
        const bool rot = a.apply != 0 && (is_q || is_k);
        f16* cache = is_q ? nullptr
                          : (is_k ? a.kc + (uint64_t)(head - Hq) * 128u
                                  : a.vc + (uint64_t)(head - Hq - Hkv) * 128u);
#pragma unroll
        for (int p = 0; p < kWBM / 64; ++p) {
            const uint32_t row = 64u * p + rsub, m = m0 + row;
            if (m >= a.M) break;
            const f16x8 x0 = lds16(lo + row * 64u + j8);
            const f16x8 x1 = lds16(hi + row * 64u + j8);
            f16x8 r0 = x0, r1 = x1;
            const uint64_t pos = (uint64_t)a.start_pos + m;
            if (rot) {
                const f16x8 cs = ld16(a.cos_t + pos * 64u + j8);
                const f16x8 sn = ld16(a.sin_t + pos * 64u + j8);
                rope_rotate8(x0, x1, cs, sn, r0, r1);
            }
            f16* yr = a.y + (uint64_t)m * N + hn0;
            if (is_q) {
                st16(yr + j8, r0);
                st16(yr + 64u + j8, r1);
            } else {
                st16(yr + j8, x0);
                st16(yr + 64u + j8, x1);
                f16* cr = cache + pos * kv_dim;
                st16(cr + j8, r0);
                st16(cr + 64u + j8, r1);
            }
        }
    }
}

// Any shape and alignment: one thread per output element, fp32 accumulation.
// Block b covers token b / n_tiles, features 256 (b % n_tiles) + 0..255.
__global__ __launch_bounds__(256) void qkv_gemm_generic(QkvGemmArgs a) {
    const uint32_t m = blockIdx.x / a.n_tiles;
    const uint32_t col = (blockIdx.x - m * a.n_tiles) * 256u + threadIdx.x;
    if (col >= a.N) return;
    const f16* xr = a.x + (uint64_t)m * a.K;
    const f16* wr = a.w + (uint64_t)col * a.K;
    float acc = 0.f;
    for (uint32_t k = 0; k < a.K; ++k) acc += (float)xr[k] * (float)wr[k];
    a.y[(uint64_t)m * a.N + col] = (f16)acc;
}

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

template <int WMT>
hipError_t launch_mfma(const QkvGemmArgs& a, bool fused, hipStream_t stream) {
    constexpr int BM = 64 * WMT;
    QkvGemmArgs b = a;
    b.n_tiles = (a.N + 127u) / 128u;
    b.vec_out = (a.N % 8u == 0 && aligned16(a.y)) ? 1u : 0u;
    const uint64_t m_tiles = (a.M + BM - 1u) / BM;
    const uint64_t blocks = m_tiles * b.n_tiles;
    if (blocks > 0x7fffffffull) return hipErrorInvalidValue;
    b.m_tiles = (uint32_t)m_tiles;
    if (fused)
        hipLaunchKernelGGL((qkv_gemm_mfma<WMT, true>), dim3((uint32_t)blocks), dim3(kThreads), 0,
                           stream, b);
    else
        hipLaunchKernelGGL((qkv_gemm_mfma<WMT, false>), dim3((uint32_t)blocks), dim3(kThreads), 0,
                           stream, b);
    return hipGetLastError();
}

hipError_t launch_wide(const QkvGemmArgs& a, bool fused, hipStream_t stream) {
    QkvGemmArgs b = a;
    b.n_tiles = a.N / kWBN;
    b.vec_out = 1u;
    b.m_tiles = (a.M + kWBM - 1u) / kWBM;
    const uint64_t blocks = (uint64_t)b.m_tiles * b.n_tiles;
    if (blocks > 0x7fffffffull) return hipErrorInvalidValue;
    if (fused)
        hipLaunchKernelGGL(qkv_gemm_wide<true>, dim3((uint32_t)blocks), dim3(kWThreads), 0, stream,
                           b);
    else
        hipLaunchKernelGGL(qkv_gemm_wide<false>, dim3((uint32_t)blocks), dim3(kWThreads), 0, stream,
                           b);
    return hipGetLastError();
}

// The wide tile needs whole 384-feature tiles and 16-byte aligned output
// rows; it pays off once there are enough token tiles to fill the CUs.
bool use_wide(const QkvGemmArgs& a) {
    const long forced = get_option(kOptQkvGemmWide);
    if (forced == 1) return false;
    if (a.N % kWBN != 0 || a.K % kWBK != 0 || !aligned16(a.y)) return false;
    return forced == 2 || a.M >= kWideMinTokens;
}

}  // namespace

bool qkv_gemm_mfma_ok(const QkvGemmArgs& a) {
    if (get_option(kOptQkvGemmForceGeneric)) return false;
    if (a.K % kBK != 0 || !aligned16(a.x) || !aligned16(a.w)) return false;
    // every row offset of X and W fits the 32-bit buffer ranges
    return (uint64_t)a.M * a.K * 2u < 0xffffffffull && (uint64_t)a.N * a.K * 2u < 0xffffffffull;
}

int qkv_gemm_wmt(uint32_t M) {
    const long forced = get_option(kOptQkvGemmTokensPerWave);
    if (forced == 32 || forced == 64 || forced == 128) return (int)(forced / 32);
    return M > 1024u ? 4 : (M > 256u ? 2 : 1);
}

hipError_t launch_qkv_gemm_kernel(const QkvGemmArgs& a, bool fused, hipStream_t stream) {
    if (a.M == 0 || a.N == 0) return hipSuccess;
    if (!qkv_gemm_mfma_ok(a)) {
        if (fused) return hipErrorInvalidValue;  // the caller runs GEMM + RoPE instead
        QkvGemmArgs b = a;
        b.n_tiles = (a.N + 255u) / 256u;
        const uint64_t blocks = (uint64_t)b.n_tiles * a.M;
        if (blocks > 0x7fffffffull) return hipErrorInvalidValue;
        hipLaunchKernelGGL(qkv_gemm_generic, dim3((uint32_t)blocks), dim3(256), 0, stream, b);
        return hipGetLastError();
    }
    if (use_wide(a)) return launch_wide(a, fused, stream);
    switch (qkv_gemm_wmt(a.M)) {
        case 1: return launch_mfma<1>(a, fused, stream);
        case 2: return launch_mfma<2>(a, fused, stream);
        default: return launch_mfma<4>(a, fused, stream);
    }
}

}  // namespace attn
