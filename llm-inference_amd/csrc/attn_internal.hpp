// Internal interface between the kernel translation units and the C-ABI layer.
// Every kernel takes ONE argument struct by value, so a captured graph node can
// be re-parameterised by copying the struct out of hipKernelNodeParams,
// editing fields and writing it back (the update_*_node entry points).
#pragma once

#include "attn_common.hpp"

namespace attn {

// ------------------------------------------------------------- RoPE + append
struct RopeArgs {
    f16* q;             // [seq, q_stride], Q heads rotated in place
    f16* k;             // [seq, k_stride] K source (rotated in place when kc == nullptr)
    const f16* v;       // [seq, k_stride] V source
    f16* kc;            // K cache rows [S][Hkv*D] or nullptr
    f16* vc;            // V cache rows [S][Hkv*D]
    const f16* cos_t;   // [S][D/2]
    const f16* sin_t;   // [S][D/2]
    uint64_t q_stride;  // elements between Q tokens
    uint64_t k_stride;  // elements between K/V source tokens
    uint32_t seq_len;
    uint32_t num_heads;
    uint32_t num_kv_heads;
    uint32_t head_dim;
    uint32_t start_pos;      // cache row / table row of token 0 (patched per decode step)
    uint32_t apply;          // 1: rotate Q and K; 0: NoPE, copy K and V only (patched)
    uint32_t lanes_per_head; // vector path: D/16 lanes per head (each lane = 8 pairs)
    uint32_t pad_;
};

// Decode-step QKV projection y = W x (fp16 in, fp32 accumulate, fp16 out),
// optionally followed in the same kernel by RoPE + KV-cache append.
struct QkvArgs {
    const f16* x;        // [in_dim]
    const f16* w;        // [out_dim][in_dim] row-major: Q rows, then K, then V
    f16* y;              // [out_dim] (fused: Q rotated, K and V as projected)
    f16* kc;             // fused: K cache rows [S][Hkv*D]
    f16* vc;             // fused: V cache rows
    const f16* cos_t;    // fused: [S][D/2]
    const f16* sin_t;
    uint32_t out_dim;
    uint32_t in_dim;
    uint32_t num_heads;
    uint32_t num_kv_heads;
    uint32_t head_dim;
    uint32_t start_pos;  // fused: cache/table row (patched per decode step)
    uint32_t apply;      // fused: 1 rotate Q and K, 0 NoPE (patched)
    float beta;          // unfused: y = W x + beta * y (the o_proj residual add); 0 for QKV
};

// Prefill QKV projection Y[M][N] = X[M][K] . W[N][K]^T (fp16 in, fp32
// accumulate, fp16 out, Y row stride N), optionally followed in the same
// kernel by RoPE + KV-cache append of the M tokens (D = 128 heads).
struct QkvGemmArgs {
    const f16* x;        // [M][K]
    const f16* w;        // [N][K]: Q rows, then K, then V
    f16* y;              // [M][N] (fused: Q rotated, K and V as projected)
    f16* kc;             // fused: K cache rows [S][Hkv*128]
    f16* vc;             // fused: V cache rows
    const f16* cos_t;    // fused: [S][64]
    const f16* sin_t;
    uint32_t M;
    uint32_t N;
    uint32_t K;
    uint32_t n_tiles;    // set by the launcher
    uint32_t num_heads;
    uint32_t num_kv_heads;
    uint32_t start_pos;  // fused: cache/table row of token 0
    uint32_t apply;      // fused: 1 rotate Q and K, 0 NoPE
    uint32_t vec_out;    // set by the launcher: 16-byte stores of y (N % 8 == 0, y aligned)
    uint32_t m_tiles;    // set by the launcher: token tiles
};

bool qkv_gemm_mfma_ok(const QkvGemmArgs& a);
int qkv_gemm_wmt(uint32_t M);
// fused: only when qkv_gemm_mfma_ok (hipErrorInvalidValue otherwise)
hipError_t launch_qkv_gemm_kernel(const QkvGemmArgs& a, bool fused, hipStream_t stream);

hipError_t launch_qkv_kernel(const QkvArgs& a, bool fused, hipStream_t stream);
const void* qkv_kernel_symbol(bool fused, bool vec);
bool qkv_vectorized(const QkvArgs& a);

hipError_t launch_rope_kernel(const RopeArgs& a, bool vector_path, hipStream_t stream);
bool rope_vector_ok(const RopeArgs& a);
const void* rope_kernel_symbol(bool vector_path);

// ------------------------------------------------------------- Flash-Decode
struct DecodeArgs {
    const f16* q;        // [Hq][D] packed
    const f16* k;        // cache rows, kv_stride elements apart
    const f16* v;
    f16* out;            // [Hq][D] packed
    float* part_out;     // [Hq][nstate][D] fp16 normalised outputs (workspace, see state_out)
    float* part_max;     // [Hq][nstate]      (workspace, log2 domain)
    float* part_sum;     // [Hq][nstate]      (workspace)
    uint64_t kv_stride;
    uint32_t kv_len;     // patched per decode step
    uint32_t num_heads;
    uint32_t num_kv_heads;
    uint32_t group;      // Hq / Hkv
    uint32_t head_dim;
    uint32_t nsplit;     // context splits per KV head (patched)
    uint32_t chunk;      // keys per split (patched)
    uint32_t nstate;     // partial states per query head (patched)
    uint32_t whole_ok;   // the caller's launch may run as one kernel (see plan_decode)
    uint32_t whole;      // one split per KV-head group: the split kernel writes the
                         // output (and q rotated), the merge kernel exits (patched)
    float scale_log2;    // log2(e) / sqrt(D)
    // fused RoPE + KV append of the decoded token (the ROPE kernel variants):
    // q rotated in registers by the split kernel and in place by the merge
    // kernel; cache row `row` of K (rotated) and V written from k_src / v_src
    // by the split workgroups whose chunk holds it, before they read it
    f16* q_rot;          // = q, writable
    f16* k_dst;          // = k, writable (cache rows kv_stride apart)
    f16* v_dst;
    const f16* k_src;    // [Hkv][D] of the new token
    const f16* v_src;
    const f16* cos_t;    // [S][D/2]
    const f16* sin_t;
    uint32_t row;        // cache row of the new token (start_pos, patched)
    uint32_t apply;      // 1: rotate q and K; 0: copy K and V only (patched)
#if defined(ATTN_DECODE_TIMELINE)
    // instrumented build (libattn_timeline.so) only: this call's record of
    // per-workgroup timestamps, set by the launchers
    uint64_t* tl;
#endif
};

#if defined(ATTN_DECODE_TIMELINE)
// Record layout of one decode call (64-bit words): split workgroup w at
// 16 w: [0] entry, [15] wave 0 about to load q, [1] its first K/V loads
// issued, [2 + wave] that
// wave's last batch computed (0: the wave had no keys), [14] every wave's
// state in LDS (after the barrier), [10] thread 0's share of the fold done
// and its partial stores issued, [11] those stores acknowledged, [12] HW_ID,
// [13] XCC_ID; merge workgroup m at kTlMergeBase + 4 m: [0] entry, [1]
// partial states loaded and folded, [2] output stored and acknowledged,
// [3] XCC_ID.  Times are s_memrealtime ticks (100 MHz).  No wait or barrier
// is added to the kernels except thread 0's wait for its own stores.
constexpr uint32_t kTlSplitWords = 16;
constexpr uint32_t kTlMaxSplitWgs = 1024;
constexpr uint32_t kTlMergeBase = kTlSplitWords * kTlMaxSplitWgs;
constexpr uint32_t kTlMaxMergeWgs = 1024;
constexpr uint32_t kTlSlotWords = kTlMergeBase + 4 * kTlMaxMergeWgs;
#endif

// The partial states' outputs: [Hq][nstate][D] fp16 at the start of the
// caller's part_out buffer, each the state's output normalised by its own
// sum (acc / l); the maxima and sums stay fp32 in part_max / part_sum.
__device__ __forceinline__ f16* state_out(const DecodeArgs& a) {
    return reinterpret_cast<f16*>(a.part_out);
}

// The fused RoPE + decode form: the split kernel leaves the new token's
// position in the word after the fp16 partial outputs, and the merge kernel
// that rotates q reads it there, so a merge node whose state count and
// rotation switch are unchanged needs no patch when the position moves.  The
// caller's partial_out holds at least num_heads * nstate * D floats, twice
// the fp16 outputs, so the word lies inside it.
__device__ __forceinline__ uint32_t* rope_row_word(const DecodeArgs& a) {
    return reinterpret_cast<uint32_t*>(state_out(a) + (uint64_t)a.num_heads * a.nstate * 128u);
}

// q head h (D = 128) at position `row` rotated in place by lanes 0..7 of the
// calling threads (lane e: pairs 8e..8e+7 and their partners 64 + 8e..), as
// launch_rope_and_store_kv leaves it; used by the merge kernels of the fused
// RoPE + decode form once every split workgroup has read q.
__device__ __forceinline__ void rotate_q_head(const DecodeArgs& a, uint32_t h, uint32_t e,
                                              uint32_t row) {
    const uint32_t c8 = 8u * e;
    f16* qh = a.q_rot + (uint64_t)h * 128u;
    f16x8 x0 = ld16(qh + c8), x1 = ld16(qh + 64 + c8);
    rope_rotate8(x0, x1, ld16(a.cos_t + (uint64_t)row * 64u + c8),
                 ld16(a.sin_t + (uint64_t)row * 64u + c8), x0, x1);
    st16(qh + c8, x0);
    st16(qh + 64 + c8, x1);
}

struct DecodePlan {
    // 0 = generic (any D, any stride); 1/2/3 = MFMA split kernel with 4/2/1 KV
    // heads per workgroup + merge kernel
    int path;
    uint32_t nsplit;
    uint32_t chunk;
    uint32_t nstate;   // partial states per query head written to the workspace
    uint32_t block;    // threads per split workgroup
    uint32_t groups;   // KV-head groups (grid of the split workgroups: nsplit x groups)
    uint32_t kdma;     // 1: the split kernel reads K through LDS-DMA in whole rows
    uint32_t whole;    // 1: one split per KV-head group and no merge work
};

// allow_whole: the launch may be one kernel for short contexts (callers that
// do not need the merge kernel's separate node)
DecodePlan plan_decode(uint32_t kv_len, uint32_t num_heads, uint32_t num_kv_heads,
                       uint32_t head_dim, uint64_t kv_stride, const void* q, const void* k,
                       const void* v, int device, bool allow_whole);
// Recompute the split/chunk fields of an argument struct for its kv_len and
// return the plan, whose path (heads per workgroup) also depends on kv_len.
// Used by launch and by the graph-node updaters (same plan for the same L):
// an updater sets the split node's kernel to the plan's path as well as its
// grid and arguments.
DecodePlan replan_decode(DecodeArgs& a, int device);
int decode_hpw(int path);                        // KV heads per split workgroup (0: generic)
dim3 decode_grid(const DecodeArgs& a, const DecodePlan& p);  // the split kernel's grid
dim3 decode_merge_grid(const DecodeArgs& a);                  // the merge kernel's grid
// Enqueues the split kernel (followed by launch_decode_merge).
hipError_t launch_decode_split(const DecodeArgs& a, const DecodePlan& p, hipStream_t stream,
                               bool rope = false);
hipError_t launch_decode_merge(const DecodeArgs& a, hipStream_t stream, bool rope = false);
const void* decode_split_symbol(const DecodePlan& p, bool rope = false);
// the merge kernel, or for a whole-context plan the kernel that does nothing
const void* decode_merge_symbol(bool rope = false, bool whole = false);
int decode_path_of_symbol(const void* fn, bool rope);  // 0 when not a split kernel

// Decode attention's partial-state merge fused into the attention output
// projection (o_proj, y = W_o attn + beta y): workgroup (head h, row block)
// merges head h's partial states into the head's fp16 attention output (the
// merge kernel's result, written to d.out by row block 0) and multiplies it by
// head h's columns of W_o for the block's rows; the fp32 products go to
// y_part[h][row].  The last workgroup of a row block to finish (an atomic
// count per block) sums the heads in order, adds beta * y and stores y in
// fp16, then clears its count for the next call.
struct OutProjArgs {
    DecodeArgs d;          // the decode's arguments (states, plan; patched with kv_len)
    const f16* w;          // W_o [hidden][num_heads * 128] row-major
    f16* y;                // [hidden]: residual in (beta != 0), projection out
    float* y_part;         // [num_heads][hidden] fp32 workspace
    uint32_t* counters;    // [row_blocks], zero before the first call (left zero)
    uint32_t hidden;
    uint32_t row_blocks;   // ceil(hidden / 128)
    float beta;
    uint32_t xcd_map;      // 1: a head's workgroups share one XCD (num_heads % 8 == 0)
};
constexpr uint32_t kOutProjRows = 128;  // W_o rows per workgroup
// workspace bytes: y_part, then the counters
size_t out_proj_workspace_bytes(size_t num_heads, size_t hidden);
bool out_proj_fused_ok(const OutProjArgs& a);
hipError_t launch_merge_out_proj(const OutProjArgs& a, hipStream_t stream, bool rope);
const void* merge_out_proj_symbol(bool rope);

// ------------------------------------------------------------- prefill
struct PrefillArgs {
    const f16* q;       // [N] rows, q_stride elements apart, Hq heads of D
    const f16* k;       // [N] rows, kv_stride apart, Hkv heads of D
    const f16* v;
    f16* out;           // packed [N][Hq][D]
    uint64_t q_stride;
    uint64_t kv_stride;
    uint32_t seq_len;
    uint32_t num_heads;
    uint32_t num_kv_heads;
    uint32_t group;
    uint32_t head_dim;
    uint32_t q_tiles;   // MFMA path: number of query tiles (set by the launcher)
    float scale_log2;
    uint32_t pad_;
};

int plan_prefill(const PrefillArgs& a);  // 0 generic, 1 MFMA
hipError_t launch_prefill_kernel(const PrefillArgs& a, int path, hipStream_t stream);

// generic attention (one workgroup per query row and head); also the decode
// fallback for head_dim != 128 or unaligned strides
struct GenericAttnArgs {
    const f16* q;
    const f16* k;
    const f16* v;
    f16* out;
    uint64_t q_stride;
    uint64_t kv_stride;
    uint32_t nq;        // query rows
    uint32_t kv_len;    // keys visible to every row (patched for decode)
    uint32_t num_heads;
    uint32_t group;
    uint32_t head_dim;
    uint32_t causal;    // 1: row t sees keys <= t (start position 0)
    float scale_log2;
    uint32_t pad_;
};
hipError_t launch_generic_attention(const GenericAttnArgs& a, hipStream_t stream);
const void* generic_attention_symbol();

// option switches for tests/benchmarks (process-wide)
enum Option {
    kOptDecodeForceGeneric = 0,
    kOptDecodeSplits = 1,        // 0 = automatic
    kOptPrefillForceGeneric = 2,
    kOptDecodeHeadsPerGroup = 3,  // 0 = automatic; 1, 2 or 4 KV heads per split workgroup
    kOptQkvGemmForceGeneric = 4,
    kOptQkvGemmTokensPerWave = 5, // 0 = automatic; 32, 64 or 128
    kOptQkvGemmWide = 6,          // 0 = automatic; 1 = never; 2 = whenever the shape allows
    kOptPrefillWaves = 7,         // 0 = automatic; 4 or 8 waves per prefill workgroup
    kOptDecodeOutProjFused = 8,   // 1: attn_decode_out_proj runs the fused merge + o_proj kernel
    kOptPrefillStageAll = 9,      // 0 = automatic (N <= 256: all key tiles staged at once); 1 = never
    kOptPrefillSplitKeys = 10,    // 0 = automatic; 1 = never; 2 = 64-key tiles over 4 waves; 3 = 32-key units over 8 waves; 4 = 32-key units streamed per wave
    kOptPrefillKeyHalves = 11,    // 0 = automatic; 1 = never; 2 = 32-query tiles whose key tiles two 4-wave groups split
    kOptDecodeKdma = 12,          // 0 = automatic; 1 = K in registers; 2 = K through LDS-DMA
    kOptGraphNodeRecords = 13,    // 0 = updaters use the nodes recorded at capture; 1 = read nodes back
    kOptDecodeWholeMaxKeys = 14,  // 0 = automatic; < 0 never; > 0 longest one-kernel context
    kOptCount = 15
};
long get_option(int which);

int device_cu_count(int device);

}  // namespace attn
