// Flash-Decode's merge fused into the attention output projection (o_proj)
// of the same decode step, for gfx950.
//
// The reference engine runs, per layer, the decode's split and merge kernels
// (the merge writes the fp16 attention output, causal_attention.hip.cpp:
// 804-852) and then launch_attention_out_projection_decode
// (attention_out_projection.hip.cpp:61-71): the GEMV y = W_o attn + beta y of
// matrix_vec_mul.hip.cpp:79-172 with beta = 1, the residual add
// (model_inference.hpp:390-397).  Here the merge and the GEMV are one kernel:
//
//   workgroup (head h, row block b) = 8 waves.  First it issues the loads of
//   its W_o block (rows 128 b .. 128 b + 127, columns 128 h .. 128 h + 127:
//   256 bytes per row, 4 rows per wave instruction), then merges head h's
//   partial states: wave w folds splits w, w + 8, ... (lanes over the 128
//   dims, 512 bytes per split per instruction), the 8 wave states combine in
//   LDS into the head's attention output, rounded to fp16 as the merge kernel
//   stores it (row block 0 also writes it to the decode's output).  The
//   products of those 128 values with the W_o block (v_dot2_f32_f16, a 16-lane
//   reduction per row) go to y_part[h][row] in fp32.  The last of the
//   num_heads workgroups of a row block to finish (an agent-scope atomic count
//   taken once the partials are stored) sums y_part over the heads in head
//   order, adds beta * y and stores y in fp16; it then clears the count, so the
//   counters are zero again for the next call or graph replay.
//
// Every head's merge is repeated by each of its row blocks (16 for hidden
// 2048): with num_heads % 8 == 0 the workgroups of one head are placed on one
// XCD (workgroups are dispatched to the 8 XCDs round-robin by linear id), so
// the states come from HBM/MALL once per head and from the XCD's L2 after.
#include "attn_internal.hpp"

namespace attn {

namespace {

constexpr uint32_t kDim = 128;
constexpr uint32_t kWaves = 8;
constexpr int kRound = 4;  // splits per wave per round of loads
constexpr uint32_t kXcds = 8;
constexpr int kSc1 = 16;  // cache-policy bit sc1 of buffer loads: device-coherent


__device__ __forceinline__ float ldf(BufRsrc r, uint32_t byte_off) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)byte_off, 0, 0));
}

template <bool ROPE>
__global__ __launch_bounds__(512) void merge_out_proj(OutProjArgs a) {
    __shared__ float s_m[kWaves];
    __shared__ float s_l[kWaves];
    __shared__ float s_acc[kWaves][kDim];
    __shared__ __attribute__((aligned(16))) f16 s_o[kDim];
    __shared__ uint32_t s_last;

    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63u;
    const uint32_t wave = (uint32_t)__builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t H = a.d.num_heads;
    const uint32_t R = a.row_blocks;
    uint32_t h, rb;
    if (a.xcd_map) {
        const uint32_t x = blockIdx.x % kXcds, slot = blockIdx.x / kXcds;
        h = x * (H / kXcds) + slot / R;
        rb = slot % R;
    } else {
        h = blockIdx.x / R;
        rb = blockIdx.x % R;
    }

    // ---- W_o block loads, issued before the merge (they do not depend on it)
    const uint32_t in_dim = H * kDim;
    const uint32_t row0 = rb * kOutProjRows;
    const uint32_t rows = min(kOutProjRows, a.hidden - row0);
    const uint32_t row_bytes = in_dim * 2u;
    // rows past `rows` fall outside the range and read zeros
    const BufRsrc rw = make_rsrc(a.w + (uint64_t)row0 * in_dim + (uint64_t)h * kDim,
                                 (rows - 1u) * row_bytes + kDim * 2u);
    const uint32_t quarter = lane >> 4, l16 = lane & 15u;
    f16x8 wv[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        const uint32_t r = (uint32_t)s * 32u + wave * 4u + quarter;
        wv[s] = buf_ld16_nt(rw, r * row_bytes + l16 * 16u);  // each weight is read once
    }

    // ---- merge of head h: wave w folds splits w, w + 8, ...; lane: dims 2l, 2l + 1
    const uint32_t S = a.d.nstate;
    const BufRsrc rpm = make_rsrc(a.d.part_max + (uint64_t)h * S, S * 4u);
    const BufRsrc rps = make_rsrc(a.d.part_sum + (uint64_t)h * S, S * 4u);
    const BufRsrc rpo = make_rsrc(state_out(a.d) + (uint64_t)h * S * kDim, S * kDim * 2u);
    float m = -INFINITY, l = 0.f;
    f32x2 acc = {0.f, 0.f};
    for (uint32_t base = wave; base < S; base += kWaves * kRound) {
        float mc[kRound], lc[kRound];
        f16x2 ac[kRound];
#pragma unroll
        for (int u = 0; u < kRound; ++u) {
            const uint32_t c = base + kWaves * (uint32_t)u;  // past S: zeros
            mc[u] = ldf(rpm, c * 4u);
            lc[u] = ldf(rps, c * 4u);
            ac[u] = __builtin_bit_cast(
                f16x2, __builtin_amdgcn_raw_buffer_load_b32(rpo, (int)(c * (kDim * 2u) + lane * 4u),
                                                            0, 0));
        }
#pragma unroll
        for (int u = 1; u < kRound; ++u)
            if (base + kWaves * (uint32_t)u >= S) mc[u] = -INFINITY;
        float mn = m;
#pragma unroll
        for (int u = 0; u < kRound; ++u) mn = fmaxf(mn, mc[u]);  // split `base` is valid
        const float so = fast_exp2(m - mn);  // first round: 2^-inf = 0
        l *= so;
        acc *= so;
#pragma unroll
        for (int u = 0; u < kRound; ++u) {
            // state c's weight 2^(m_c - M) l_c times its normalised output
            const float wc = fast_exp2(mc[u] - mn) * lc[u];  // invalid splits: 0
            l += wc;
            acc.x += (float)ac[u][0] * wc;
            acc.y += (float)ac[u][1] * wc;
        }
        m = mn;
    }
    // waves without splits (S < 8) keep m = -inf and get weight 0 below
    if (lane == 0) {
        s_m[wave] = m;
        s_l[wave] = l;
    }
    s_acc[wave][2u * lane] = acc.x;
    s_acc[wave][2u * lane + 1u] = acc.y;
    __syncthreads();
    if (tid < kDim) {
        float M = s_m[0];
#pragma unroll
        for (uint32_t w = 1; w < kWaves; ++w) M = fmaxf(M, s_m[w]);
        float num = 0.f, den = 0.f;
#pragma unroll
        for (uint32_t w = 0; w < kWaves; ++w) {
            const float sc = fast_exp2(s_m[w] - M);
            den += s_l[w] * sc;
            num += s_acc[w][tid] * sc;
        }
        const f16 o = (f16)(num / den);
        s_o[tid] = o;
        if (rb == 0) a.d.out[(uint64_t)h * kDim + tid] = o;
    }
    if constexpr (ROPE) {
        // every split workgroup has read q (the kernel boundary orders this)
        if (rb == 0 && a.d.apply && tid < 8u) rotate_q_head(a.d, h, tid, a.d.row);
    }
    __syncthreads();

    // ---- head h's share of the block's rows: 16 lanes per row, 8 dims per lane
    const f16x8 xo = *reinterpret_cast<const f16x8*>(&s_o[l16 * 8u]);
    float p[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        p[s] = 0.f;
#pragma unroll
        for (int e = 0; e < 8; e += 2)
            p[s] = __builtin_amdgcn_fdot2(f16x2{wv[s][e], wv[s][e + 1]}, f16x2{xo[e], xo[e + 1]},
                                          p[s], false);
    }
#pragma unroll
    for (int o = 8; o >= 1; o >>= 1)
#pragma unroll
        for (int s = 0; s < 4; ++s) p[s] += xor_lane(p[s], o);
    // lane s of each 16-lane group stores row s * 32 + 4 wave + quarter.  The
    // partials, the count and the last workgroup's reads of them are
    // agent-scope atomic accesses: they are coherent across the XCDs' L2s
    // without a release fence (which would write back the whole L2 of the
    // XCD once per workgroup)
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        const uint32_t r = (uint32_t)s * 32u + wave * 4u + quarter;
        if (l16 == (uint32_t)s && r < rows)
            __hip_atomic_store(&a.y_part[(uint64_t)h * a.hidden + row0 + r], p[s],
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }

    // ---- the last workgroup of the row block sums the heads
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's partials are stored
    __syncthreads();
    if (tid == 0)
        s_last = __hip_atomic_fetch_add(&a.counters[rb], 1u, __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_AGENT) == H - 1u ? 1u : 0u;
    __syncthreads();
    if (s_last == 0u) return;  // workgroup-uniform
    // Ordering of the hand-off.  The HIP memory model would need a release on
    // the count and an acquire here; at agent scope on gfx950 those are L2
    // write-back / invalidate operations for the whole XCD, paid once per
    // workgroup.  Instead every partial is an agent-scope atomic store (a
    // device-coherent store, sc1), each wave waits for its own stores to
    // complete (s_waitcnt vmcnt(0): the store is acknowledged by the device
    // coherence point) before the barrier and the count, and the last
    // workgroup reads the partials with device-coherent loads (sc1, below),
    // which do not hit stale L2 lines.  This relies on the hardware behaviour
    // just described (completed sc1 stores are visible to sc1 loads from any
    // XCD), not on the language model; the workgroup-scope acquire keeps the
    // compiler from moving those loads above the count.
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    if (tid < rows) {
        // device-coherent loads (cache-policy bit sc1, as agent-scope atomic
        // loads are issued) of the heads' partials, 8 in flight, summed in
        // head order; rows past the range read zeros
        const BufRsrc ryp = make_rsrc(a.y_part, H * a.hidden * 4u);
        const uint32_t off = (row0 + tid) * 4u;
        float sum = 0.f;
        for (uint32_t h0 = 0; h0 < H; h0 += 8u) {
            float v[8];
#pragma unroll
            for (uint32_t u = 0; u < 8u; ++u)
                v[u] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                     ryp, (int)((h0 + u) * a.hidden * 4u + off),
                                                     0, kSc1));
#pragma unroll
            for (uint32_t u = 0; u < 8u; ++u) sum += v[u];  // heads past H read 0
        }
        // matrix_vec_mul.hip.cpp:156-163: the fp32 sum plus beta * y, rounded once
        if (a.beta != 0.f) sum += a.beta * (float)a.y[row0 + tid];
        a.y[row0 + tid] = (f16)sum;
    }
    if (tid == 0) __hip_atomic_store(&a.counters[rb], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

size_t out_proj_workspace_bytes(size_t num_heads, size_t hidden) {
    const size_t part = (num_heads * hidden * sizeof(float) + 255) & ~(size_t)255;
    const size_t blocks = (hidden + kOutProjRows - 1) / kOutProjRows;
    return part + blocks * sizeof(uint32_t);
}

bool out_proj_fused_ok(const OutProjArgs& a) {
    const auto a16 = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
    const uint64_t in_dim = (uint64_t)a.d.num_heads * kDim;
    return a.d.head_dim == kDim && a.d.num_heads > 0 && a.hidden > 0 && a16(a.w) &&
           ((uintptr_t)a.counters & 3u) == 0 && ((uintptr_t)a.y_part & 3u) == 0 &&
           // W_o block offsets within 32 bits; state ranges as the merge kernel needs
           (uint64_t)kOutProjRows * in_dim * 2u < 0x80000000ull &&
           ((uint64_t)a.d.num_heads + 8u) * a.hidden * 4u < 0x80000000ull &&
           (uint64_t)a.d.num_heads * a.row_blocks < 0x80000000ull;
}

const void* merge_out_proj_symbol(bool rope) {
    return rope ? reinterpret_cast<const void*>(&merge_out_proj<true>)
                : reinterpret_cast<const void*>(&merge_out_proj<false>);
}

hipError_t launch_merge_out_proj(const OutProjArgs& a, hipStream_t stream, bool rope) {
    void* args[1] = {const_cast<OutProjArgs*>(&a)};
    return hipLaunchKernel(merge_out_proj_symbol(rope), dim3(a.d.num_heads * a.row_blocks),
                           dim3(512), args, 0, stream);
}

}  // namespace attn
